"""CPU checks of libsmoe.so: it loads without a GPU, exports every entry
point include/smoe.h declares, and its host-side argument validation and
workspace layout behave (no kernel is launched here)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "smoe.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"SMOE_API\s+[\w\s\*]+?\b(smoe_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def nat():
    from spider_moe_amd import _native
    if not os.path.exists(_native.LIB_PATH):
        pytest.fail("libsmoe.so is not built (run __graft_entry__.build())")
    _native.lib()
    return _native


def test_exports_every_declared_symbol(nat):
    syms = declared_symbols()
    assert len(syms) >= 14
    handle = ctypes.CDLL(nat.LIB_PATH)
    for s in syms:
        assert hasattr(handle, s), s
    # and the Python binding covers exactly the declared set
    assert set(nat.SIGNATURES) == set(syms)


def test_identity(nat):
    lib = nat.lib()
    assert lib.smoe_abi_version() == 4
    assert lib.smoe_backend_name() == b"hip-gfx950"
    assert lib.smoe_backend_caps() == 0b1111


def _block(nat, **kw):
    b = nat.SmoeBlock()
    b.act_dtype, b.H, b.E, b.K, b.M, b.L, b.R = nat.BF16, 1024, 16, 2, 2, 32, 6
    fake = 0x1000
    b.router_w = b.loop_bias = b.edge_gen_w = b.edge_loop_bias = b.edge_value_w = fake
    ex = b.experts
    ex.format, ex.act, ex.E, ex.H, ex.U = nat.BF16, nat.ACT_SWIGLU, 16, 1024, 2816
    ex.w_up = ex.w_down = fake
    b.alpha, b.beta, b.eps = 0.5, 0.1, 1e-5
    for k, v in kw.items():
        if hasattr(ex, k) and k in ("format", "act", "U", "group_size", "scale_dtype"):
            setattr(ex, k, v)
        else:
            setattr(b, k, v)
    return b


def test_workspace_layout_is_consistent(nat):
    lib = nat.lib()
    b = _block(nat)
    n = 16384
    lay = nat.SmoeWsLayout()
    assert lib.smoe_block_workspace_layout(ctypes.byref(b), n, ctypes.byref(lay)) == 0
    assert lay.total == lib.smoe_block_workspace_bytes(ctypes.byref(b), n)
    offs = sorted((getattr(lay, f), f) for f in nat._LAYOUT_FIELDS if f != "total")
    assert all(o % 256 == 0 for o, _ in offs)
    assert lay.front == lay.total  # the fused small-step front is off at this N: empty region
    assert max(o for o, f in offs if f != "front") < lay.total
    assert lay.S == 4 and lay.ffn_dtype == nat.BF16
    # regions do not overlap: each is at least its size from the next
    assert lay.top_idx - lay.logits >= n * 16 * 4
    assert lay.act + n * 2 * 2816 * 2 <= lay.y
    assert lay.proj + n * 4 * 1024 * 2 <= lay.msg
    # a decode-size step (N <= 256, bf16) gets the front region: [N, E + E*E] f32
    small = nat.SmoeWsLayout()
    assert lib.smoe_block_workspace_layout(ctypes.byref(b), 64, ctypes.byref(small)) == 0
    assert small.total - small.front >= 64 * (16 + 16 * 16) * 4


@pytest.mark.parametrize("bad", [dict(K=0), dict(K=17), dict(E=65), dict(M=0), dict(H=1000),
                                 dict(act_dtype=7), dict(format=9), dict(U=100),
                                 dict(format=3, group_size=48)])
def test_invalid_block_is_rejected_without_launch(nat, bad):
    lib = nat.lib()
    b = _block(nat, **bad)
    if "E" in bad:
        b.experts.E = bad["E"]
    assert lib.smoe_block_workspace_bytes(ctypes.byref(b), 64) == 0
    rc = lib.smoe_block_forward(ctypes.byref(b), 0x1000, 0x1000, 0x1000, 64, 0, 1, 0x1000, 1 << 40, None)
    assert rc in (1, -2)
    assert lib.smoe_last_error()


def test_pack_weight_tiles_rejects_bad_shapes(nat):
    lib = nat.lib()
    for g, n, k in [(0, 16, 64), (1, 10, 64), (1, 16, 100), (1, 8, 64)]:
        for code in (nat.BF16, nat.FP8_E4M3):
            assert lib.smoe_pack_weight_tiles(0x1000, code, g, n, k, 0x2000, None) == 1
    assert lib.smoe_pack_weight_tiles(None, nat.BF16, 1, 16, 64, 0x2000, None) == 1
    assert lib.smoe_pack_weight_tiles(0x1008, nat.BF16, 1, 16, 64, 0x2000, None) == 1  # alignment
    for code in (nat.F32, nat.INT4, nat.F16):  # formats without a tile layout
        assert lib.smoe_pack_weight_tiles(0x1000, code, 1, 16, 64, 0x2000, None) == -2


def test_capacity_and_range_errors(nat):
    lib = nat.lib()
    b = _block(nat)
    need = lib.smoe_block_workspace_bytes(ctypes.byref(b), 64)
    rc = lib.smoe_block_forward(ctypes.byref(b), 0x1000, 0x1000, 0x1000, 64, 0, 1, 0x1000, need - 1, None)
    assert rc == 3
    rc = lib.smoe_block_forward(ctypes.byref(b), 0x1000, 0x1000, 0x1000, 64, 5, 2, 0x1000, need, None)
    assert rc == 1  # loop range past num_loops
    # N == 0 is a no-op
    assert lib.smoe_block_forward(ctypes.byref(b), None, None, None, 0, 0, 1, None, 0, None) == 0
