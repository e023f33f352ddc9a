"""The .spiderw native weight bundle (spider_infer/orbit/weight_loader.py).

A bundle is an 80-byte header followed by sections:

  header   b"SPIDERW1", then 14 little-endian uint32 (version, flags, vocab,
           hidden, heads, experts, top_k, edges_per_expert, loops,
           expert_ffn, prelude layers, coda layers, 2 reserved), a uint64 at
           byte 64 (0) and the body length as a uint64 at byte 72.
           flags: 1 fp16 weights, 2 CSR graph present, 4 tied embeddings.
  section  uint32 id, uint32 dtype id, uint64 payload bytes, uint32 rank,
           4 x uint32 dims (unused ones 1), then the payload (C order).
           Id 200 is a named section: uint16 name length, utf-8 name, data.

Section ids and dtype ids are the reference's (weight_loader.py:15-38), so
bundles written by either side read on the other.  numpy only, no torch.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

MAGIC = b"SPIDERW1"
HEADER_BYTES = 80
NAMED_SECTION = 200
SECTION_IDS = {
    "token_emb": 1, "lm_head": 2, "router": 30, "loop_bias": 31, "loop_embedding": 32,
    "edge_generator": 33, "edge_value": 34, "expert_up": 35, "expert_down": 36,
    "moe_norm": 37, "exit_head": 38, "csr_row_ptr": 40, "csr_col_idx": 41, "csr_edge_w": 42,
}
SECTION_NAMES = {v: k for k, v in SECTION_IDS.items()}
DTYPES = {0: np.float32, 1: np.float16, 2: np.float16, 3: np.int32, 4: np.int8}
_META_FIELDS = ("version", "flags", "vocab_size", "hidden_size", "num_heads", "num_experts",
                "top_k", "edges_per_expert", "num_loops", "expert_ffn_size",
                "num_prelude_layers", "num_coda_layers")


@dataclass
class SpiderWMeta:
    version: int = 1
    flags: int = 0
    vocab_size: int = 0
    hidden_size: int = 0
    num_heads: int = 0
    num_experts: int = 0
    top_k: int = 0
    edges_per_expert: int = 0
    num_loops: int = 0
    expert_ffn_size: int = 0
    num_prelude_layers: int = 0
    num_coda_layers: int = 0

    @property
    def fp16_weights(self) -> bool:
        return bool(self.flags & 1)

    @property
    def has_csr(self) -> bool:
        return bool(self.flags & 2)

    @property
    def tied_embeddings(self) -> bool:
        return bool(self.flags & 4)


@dataclass
class SpiderWBundle:
    meta: SpiderWMeta
    tensors: dict = field(default_factory=dict)
    csr: dict | None = None
    path: str | None = None

    def require(self, name: str) -> np.ndarray:
        if name not in self.tensors:
            raise KeyError(f"missing section {name}")
        return self.tensors[name]


def _dtype_id(arr: np.ndarray) -> tuple[np.ndarray, int]:
    if arr.dtype == np.float32:
        return arr, 0
    if arr.dtype == np.float16:
        return arr, 1
    if arr.dtype == np.int32:
        return arr, 3
    if arr.dtype == np.int8:
        return arr, 4
    return arr.astype(np.float32), 0


def write_spiderw(path, meta: SpiderWMeta, tensors: dict) -> None:
    """Write a bundle: known names as numbered sections, others as named ones."""
    parts = []
    for name, arr in tensors.items():
        arr, did = _dtype_id(np.ascontiguousarray(arr))
        rank = min(arr.ndim, 4)
        dims = list(arr.shape[:4]) + [1] * (4 - rank)
        payload = arr.tobytes(order="C")
        sid = SECTION_IDS.get(name)
        if sid is None:
            nb = name.encode("utf-8")
            payload = struct.pack("<H", len(nb)) + nb + payload
            sid = NAMED_SECTION
        parts.append(struct.pack("<IIQI", sid, did, len(payload), rank))
        parts.append(struct.pack("<4I", *(int(d) for d in dims)))
        parts.append(payload)
    body = b"".join(parts)
    head = bytearray(HEADER_BYTES)
    head[:8] = MAGIC
    struct.pack_into("<14I", head, 8, *(int(getattr(meta, f)) for f in _META_FIELDS), 0, 0)
    struct.pack_into("<Q", head, 64, 0)
    struct.pack_into("<Q", head, 72, len(body))
    Path(path).write_bytes(bytes(head) + body)


def load_spiderw(path) -> SpiderWBundle:
    """Read a bundle; a truncated or unknown trailing section ends the read
    (as the reference's loader does)."""
    data = Path(path).read_bytes()
    if len(data) < HEADER_BYTES:
        raise ValueError("file too small for a spiderw header")
    if data[:8] != MAGIC:
        raise ValueError(f"bad magic: {data[:8]!r}")
    vals = struct.unpack_from("<14I", data, 8)
    meta = SpiderWMeta(**dict(zip(_META_FIELDS, vals[:12])))
    off = HEADER_BYTES
    tensors = {}
    while off + 36 <= len(data):
        sid, did, nbytes, rank = struct.unpack_from("<IIQI", data, off)
        dims = struct.unpack_from("<4I", data, off + 20)
        off += 36
        if off + nbytes > len(data) or did not in DTYPES:
            break
        raw = data[off:off + nbytes]
        off += nbytes
        dt = np.dtype(DTYPES[did])
        shape = tuple(d for d in dims[:max(rank, 1)] if d > 0)
        if sid == NAMED_SECTION:
            if len(raw) < 2:
                break
            (nlen,) = struct.unpack_from("<H", raw, 0)
            name = raw[2:2 + nlen].decode("utf-8")
            raw = raw[2 + nlen:]
        else:
            name = SECTION_NAMES.get(sid, f"section_{sid}")
        shape = shape or (len(raw) // dt.itemsize,)
        tensors[name] = np.frombuffer(raw, dtype=dt).reshape(shape).copy()
    csr = None
    keys = ("csr_row_ptr", "csr_col_idx", "csr_edge_w")
    if meta.has_csr or all(k in tensors for k in keys):
        csr = {"row_ptr": tensors.get(keys[0]), "col_idx": tensors.get(keys[1]),
               "edge_w": tensors.get(keys[2])}
    if meta.tied_embeddings and "lm_head" not in tensors and "token_emb" in tensors:
        tensors["lm_head"] = tensors["token_emb"]
    return SpiderWBundle(meta=meta, tensors=tensors, csr=csr, path=str(path))


__all__ = ["SpiderWMeta", "SpiderWBundle", "load_spiderw", "write_spiderw", "SECTION_IDS"]
