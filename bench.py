"""Spider-MoE block throughput on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workloads c1,c2,c3,c4] [--no-cpu]

A step is one full block call (all num_loops loops back to back, one native
call) over one batch of synthetic, HBM-resident hidden states.  The headline
(`value`) is the c1 prefill workload: bf16, H 1024, E 16, top-k 2, edges 2,
U 2816 SwiGLU, 6 loops, 16384 tokens.  The other workloads are reported under
"workloads".  Prints ONE JSON line.

Roofline: the dominant kernel of each workload (the expert up / gate GEMM) is
timed with HIP events around its launches (on the stream the kernels run on)
inside the timed region; achieved = algorithmic flops (prefill, MFMA-bound)
or algorithmic bytes (decode, HBM-bound) per launch / its average duration.
A second pass of the same K steps times every stage (stage_ms_per_step).
`traffic` is the HBM bytes per launch of that kernel measured with rocprofv3
--pmc FETCH_SIZE and WRITE_SIZE (scaled by the same counters' reading of a
plain copy, `--copy-calibration`), read from profiles/hbm_traffic.md.  Algorithmic work follows the per-token / per-loop accounting of
the block: F_t = 2HE + 2(H+L)Ek + 2H^2|D_t| + c H U |S_t| (c = 4 GELU, 6
SwiGLU), with |D_t| / |S_t| counted from the run's own routing.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "spider-web-moe_amd"))

PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
METRIC = "Spider-MoE block tokens/s (decode & prefill), % of HBM/MFMA roofline"

DESC = {
    "c1": "prefill bf16: H1024 E16 k2 m2 U2816 SwiGLU R6 N16384 (8x2048)",
    "c2": "decode fp8-e4m3 experts (per-channel fp32 scales): c1 block, N64 (64x1) R6",
    "c3": "skewed prefill bf16: H1024 E32 k4 m2 U1408 GELU R4 N16384, Zipf(1.2) loop bias, 4 empty experts",
    "c4": "int4 experts g128 fp16 scales: H2048 E64 k2 m4 U1408 GELU R4 N2176 (128 decode + 2048 prefill)",
}
BOUND = {"c1": "mfma", "c2": "hbm", "c3": "mfma", "c4": "hbm"}
# the GEMM stages of a loop; the roofline reports the one with the most time
GEMM_STAGES = ("edge_gemm", "up_gemm", "down_gemm")
# the kernel the launcher picks for each workload's GEMM shapes (rows per
# group, N_out, format); rocprof summaries under profiles/ name them too
GEMM_KERNEL = {
    ("c1", "up_gemm"): "k_gemm_pp<4,4,SwiGLU,320> (bf16 weight tiles, 8-wave ping-pong, LDS-DMA ring)",
    ("c1", "down_gemm"): "k_gemm_pp<4,4,down,320> (bf16 weight tiles, activations in the row-tile layout, 8-wave ping-pong, LDS-DMA ring)",
    ("c1", "edge_gemm"): "k_gemm_pp<4,4,rowscale,256> (bf16 weight tiles, 8-wave ping-pong, LDS-DMA ring)",
    ("c2", "up_gemm"): "k_gemm_decode<fp8,SwiGLU,4,1,2,3> (weight streaming, K split over 2 waves, 3-step register ring per wave)",
    ("c2", "down_gemm"): "k_gemm_decode<fp8,down,4,1,4,3> (weight streaming, K split over 4 waves)",
    ("c2", "edge_gemm"): "k_decode_edge<2,4> (bf16 weight tiles, rows found from the front's selections, K split over 4 waves; the loop's plans in workgroup 0)",
    ("c3", "up_gemm"): "k_gemm_ring<128,3,4> (bf16 GELU, LDS-DMA ring, 2 workgroups/CU)",
    ("c3", "down_gemm"): "k_gemm_pp<4,4,down,320> (bf16 weight tiles, 8-wave ping-pong)",
    ("c3", "edge_gemm"): "k_gemm_pp<4,4,rowscale,256> (bf16 weight tiles, 8-wave ping-pong)",
    ("c4", "up_gemm"): "k_gemm_stream4<GELU,6,3,3> (int4 weight streaming, 192-channel strips, dequant beside the MFMAs, LDS-DMA ring, 2 workgroups/CU)",
    ("c4", "down_gemm"): "k_gemm_stream4<down,6,3,4> (int4 weight streaming, 256-channel strips, dequant beside the MFMAs, 2 workgroups/CU)",
    ("c4", "edge_gemm"): "k_gemm_pp<4,4,rowscale,320> (bf16 weight tiles, 320-row tiles: one per destination)",
}
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.md")


def measured_traffic(name, stage):
    """HBM bytes per launch of a workload's GEMM stage from the committed pmc
    summary: lines `traffic <workload> <stage> <bytes>` (None when not
    measured)."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                parts = line.strip().strip("`").split()
                if len(parts) == 4 and parts[0] == "traffic" and parts[1:3] == [name, stage]:
                    return float(parts[3])
    except OSError:
        pass
    return None


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def expert_bytes(layer, e_touched: int) -> float:
    """Storage bytes of the touched experts' weights + scales + biases."""
    h, u = layer.hidden_size, layer.expert_ffn_size
    nup = 2 * u if layer.expert_activation == "swiglu" else u
    fmt = layer.expert_format
    n_w = nup * h + h * u
    if fmt == "fp8":
        per = n_w + 4 * (nup + h)
    elif fmt == "int4":
        g = layer._int4_w_up.group_size
        sb = layer._int4_w_up.scales.element_size()
        per = n_w / 2 + sb * (n_w / g)
    elif fmt == "bf16":
        per = 2 * n_w
    else:
        per = 4 * n_w
    if layer.expert_activation == "gelu":
        per += 4 * (u + h)
    return per * e_touched


def up_gemm_bytes(layer, rows: int, e_touched: int) -> float:
    h, u = layer.hidden_size, layer.expert_ffn_size
    nup = 2 * u if layer.expert_activation == "swiglu" else u
    fmt = layer.expert_format
    wb = {"fp8": 1.0, "int4": 0.5, "bf16": 2.0, "f32": 4.0}[fmt] * nup * h
    if fmt == "fp8":
        wb += 4 * nup
    elif fmt == "int4":
        wb += layer._int4_w_up.scales.element_size() * nup * h / layer._int4_w_up.group_size
    if layer.expert_activation == "gelu":
        wb += 4 * u
    return wb * e_touched + rows * h * 2 + rows * u * 2


def down_gemm_bytes(layer, rows: int, e_touched: int) -> float:
    h, u = layer.hidden_size, layer.expert_ffn_size
    fmt = layer.expert_format
    wb = {"fp8": 1.0, "int4": 0.5, "bf16": 2.0, "f32": 4.0}[fmt] * h * u
    if fmt == "fp8":
        wb += 4 * h
    elif fmt == "int4":
        wb += layer._int4_w_down.scales.element_size() * h * u / layer._int4_w_down.group_size
    if layer.expert_activation == "gelu":
        wb += 4 * h
    return wb * e_touched + rows * u * 2 + rows * h * 2


def gemm_work(layer, stage, acc):
    """Algorithmic (flops, bytes) of one launch of a GEMM stage, averaged
    over the loops: flops 2 H^2 per destination row (edge), 4 H U (SwiGLU) /
    2 H U (GELU) per expert row (up), 2 H U per expert row (down); bytes the
    weights of the touched groups in storage format (+ scales, biases) and
    the activation rows in and out (bf16)."""
    h, u = layer.hidden_size, layer.expert_ffn_size
    upc = 4 if layer.expert_activation == "swiglu" else 2
    f = b = 0.0
    for a in acc:
        if stage == "edge_gemm":
            f += 2 * h * h * a["d_rows"]
            b += a["d_touched"] * 2 * h * h + a["d_rows"] * h * 2 * 2
        elif stage == "up_gemm":
            f += upc * h * u * a["s_rows"]
            b += up_gemm_bytes(layer, a["s_rows"], a["e_touched"])
        else:
            f += 2 * h * u * a["s_rows"]
            b += down_gemm_bytes(layer, a["s_rows"], a["e_touched"])
    return f / len(acc), b / len(acc)


def accounting(layer, h, x0):
    """Per loop: rows with weight > 0 (sum |S_t|), destination rows
    (sum |D_t|), experts / destinations touched — from a per-loop replay
    (the kernels are deterministic, so the routing is that of the timed run)."""
    import torch
    per = []
    cur = h
    with torch.no_grad():
        for r in range(layer.num_loops):
            cur = layer(cur, x0, r)
            rt = layer.last_routing()
            per.append(dict(s_rows=int(rt["e_acnt"].sum()), d_rows=int(rt["d_cnt"].sum()),
                            e_touched=int((rt["e_acnt"] > 0).sum()),
                            d_touched=int((rt["d_cnt"] > 0).sum()),
                            counts=rt["e_acnt"].cpu().tolist()))
    return per


def block_work(layer, n, acc):
    h, e, k, lemb, u = (layer.hidden_size, layer.num_experts, layer.top_k, layer.loop_embed_size,
                        layer.expert_ffn_size)
    c = 6 if layer.expert_activation == "swiglu" else 4
    flops = bytes_ = 0.0
    for a in acc:
        flops += n * 2 * h * e + n * 2 * (h + lemb) * e * k + 2 * h * h * a["d_rows"] + c * h * u * a["s_rows"]
        bytes_ += (expert_bytes(layer, a["e_touched"]) + a["d_touched"] * 2 * h * h + 2 * h * e
                   + 2 * (h + lemb) * e * e + 2 * e * e + 4 * h + 3 * n * h * 2)
    return flops, bytes_


def run_workload(name, steps, warmup):
    import torch
    from spider_moe_amd import _native as nat
    from spider_moe_amd.workloads import make_block

    log(name, "building")
    wl = make_block(name)
    layer, h, x0 = wl.layer, wl.h, wl.x0
    n = h.shape[0] * h.shape[1]
    r = layer.num_loops
    with torch.no_grad():
        for _ in range(warmup):
            layer.forward_loops(h, x0, 0, r)
        torch.cuda.synchronize()
        log(name, "timing", steps, "steps")
        # pass 1, the timed region: K plain steps between two events
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record()
        for _ in range(steps):
            out = layer.forward_loops(h, x0, 0, r)
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = e0.elapsed_time(e1) / steps
        # pass 2: HIP events around every stage launch (breakdown), which
        # names the dominant GEMM
        timer = nat.StageTimer(capacity=steps * r * len(nat.STAGES) + 16)
        timer.start()
        for _ in range(steps):
            layer.forward_loops(h, x0, 0, r)
        stages = timer.stop()
        timer.close()
        dom = max(GEMM_STAGES, key=lambda s: sum(stages.get(s, [0.0])))
        # pass 3: the dominant GEMM alone, its launches recording their own
        # events (hipExtLaunchKernelGGL: the interval is the kernel's
        # execution); those launches cost the host ~15 us each, so the step
        # time comes from pass 1
        dom_timer = nat.StageTimer(stages=[dom], capacity=steps * r + 16, clock=True)
        dom_timer.start()
        for _ in range(steps):
            layer.forward_loops(h, x0, 0, r)
        dom_ms_list = dom_timer.stop().get(dom, [])
        sclk = dom_timer.sclk_mhz()
        dom_timer.close()
        # pass 4 (weight-streaming GEMMs): the same launches with the 256 MB
        # Infinity Cache (MALL) evicted before every loop by a 1 GiB read, so
        # their weights come from DRAM; each loop runs alone on the input the
        # chained run gave it (same routing, same touched experts)
        cold_ms_list = []
        if BOUND[name] == "hbm":
            ins = [h]
            for rr in range(r - 1):
                ins.append(layer.forward_loops(ins[-1], x0, rr, 1))
            flush = torch.ones(1 << 28, dtype=torch.float32, device=h.device)
            cold_timer = nat.StageTimer(stages=[dom], capacity=steps * r + 16)
            cold_timer.start()
            for _ in range(max(2, steps // 4)):
                for rr in range(r):
                    flush.sum()
                    layer.forward_loops(ins[rr], x0, rr, 1)
            cold_ms_list = cold_timer.stop().get(dom, [])
            cold_timer.close()
            del flush, ins
    acc = accounting(layer, h, x0)
    flops, bytes_ = block_work(layer, n, acc)
    dom_ms = sum(dom_ms_list) / max(len(dom_ms_list), 1)
    g_flops, g_bytes = gemm_work(layer, dom, acc)
    # the GEMM's bound follows its arithmetic intensity against the ridge point
    g_bound = "mfma" if g_flops / g_bytes > PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9) else "hbm"
    if g_bound == "mfma":
        ach = g_flops / (dom_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(ach / PEAK_BF16_TFLOPS, 4)}
    else:
        ach = g_bytes / (dom_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_HBM_GBS, 4)}
    roof.update({"traffic": measured_traffic(name, dom), "stage": dom,
                 "kernel": GEMM_KERNEL.get((name, dom), dom),
                 "work_per_launch": f"{g_flops:.4g} flop, {g_bytes:.4g} B",
                 "avg_launch_ms": round(dom_ms, 4)})
    if sclk is not None:
        # the shader clock of the kernel's tiles (in-kernel s_memtime against
        # the 100 MHz s_memrealtime); the peak assumes 2400 MHz
        roof["sclk_mhz"] = round(sclk, 1)
    if cold_ms_list:
        cold_ms = sum(cold_ms_list) / len(cold_ms_list)
        cold = g_bytes / (cold_ms * 1e-3) / 1e9
        roof["dram"] = {"achieved": round(cold, 1), "frac": round(cold / PEAK_HBM_GBS, 4),
                        "avg_launch_ms": round(cold_ms, 4),
                        "how": "MALL evicted (1 GiB read) before each loop: weights from DRAM"}
    if BOUND[name] == "mfma":
        blk = flops / (ms * 1e-3) / 1e12
        block_roof = {"bound": "mfma", "achieved": round(blk, 1), "unit": "TFLOP/s",
                      "frac": round(blk / PEAK_BF16_TFLOPS, 4), "work_per_step": f"{flops:.4g} flop"}
    else:
        blk = bytes_ / (ms * 1e-3) / 1e9
        block_roof = {"bound": "hbm", "achieved": round(blk, 1), "unit": "GB/s",
                      "frac": round(blk / PEAK_HBM_GBS, 4), "work_per_step": f"{bytes_:.4g} B"}
    stage_ms = {k: round(sum(v) / steps, 4) for k, v in stages.items()}
    res = {
        "workload": name, "desc": DESC[name], "tokens": n, "loops": r,
        "ms_per_step": round(ms, 4), "wall_s": round(wall, 3),
        "tokens_per_s": round(n / (ms * 1e-3), 1),
        "roofline": roof, "block_roofline": block_roof, "stage_ms_per_step": stage_ms,
        "routing": {"rows_per_loop": [a["s_rows"] for a in acc],
                    "dest_rows_per_loop": [a["d_rows"] for a in acc],
                    "expert_counts_loop0": acc[0]["counts"]},
        "checksum": float(out.float().abs().sum()),
    }
    del wl, layer, out
    torch.cuda.empty_cache()
    return res


def cpu_baseline(name="c1", sample_tokens=8192, budget_s=30.0):
    """The oracle's faithful restatement (dense edge projection, per-expert
    masks, fp32 math on the bf16-valued weights) on the host cores."""
    import torch
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from _helpers import oracle_weights  # noqa: E402
    from oracle import block as OB  # noqa: E402
    from spider_moe_amd.workloads import make_block

    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    threads = max(1, min(threads, os.cpu_count() or 1))
    torch.set_num_threads(threads)
    wl = make_block(name, device="cpu")
    w = oracle_weights(wl.layer)
    n = min(sample_tokens, wl.h.shape[0])
    h = wl.h.reshape(-1, wl.layer.hidden_size)[:n].float()
    x0 = wl.x0.reshape(-1, wl.layer.hidden_size)[:n].float()
    OB.block_loops(h[:32], x0[:32], w, 1, out_bf16=True)  # warm-up
    runs, t = 0, 0.0
    while runs < 3 and (runs == 0 or t < budget_s / 2):
        t0 = time.perf_counter()
        OB.block_loops(h, x0, w, wl.layer.num_loops, out_bf16=True)
        t += time.perf_counter() - t0
        runs += 1
    return {"value": round(n * runs / t, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{n} tokens x {wl.layer.num_loops} loops of {name}, {runs} run(s), "
                      "oracle faithful fp32 (torch CPU)"}


def run_decode_exit(steps, warmup):
    """The c2 decode step (64 tokens, 6 loops) with the early-exit gate:
    eager calls and HIP-graph replays (spider_moe_amd.graph), ungated and
    gated.  Threshold 1.0 keeps every token in orbit (the gate's own cost);
    a random exit head at threshold 0.5 makes tokens leave at mixed loops."""
    import torch
    from spider_moe_amd.graph import BlockDecodeGraph
    from spider_moe_amd.workloads import make_block

    log("decode exit: building")
    wl = make_block("c2")
    layer, h, x0 = wl.layer, wl.h, wl.x0
    hid = layer.hidden_size

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return round(e0.elapsed_time(e1) / steps, 4)

    res = {"workload": "c2 decode with the exit gate", "steps": steps}
    with torch.no_grad():
        runner = BlockDecodeGraph(layer)
        res["eager_ms"] = timed(lambda: layer.forward_loops(h, x0))
        res["graph_ms"] = timed(lambda: runner.run(h, x0, early_exit=False))
        res["eager_gate_ms"] = timed(lambda: layer.forward_loops_exit(h, x0, 1.0))
        res["graph_gate_ms"] = timed(lambda: runner.run(h, x0, early_exit=True, threshold=1.0))
        g = torch.Generator().manual_seed(31)
        layer.exit_head.weight.copy_((torch.randn(1, hid, generator=g) / hid ** 0.5).to(layer.exit_head.weight))
        layer.exit_head.bias.zero_()
        res["graph_mixed_exit_ms"] = timed(lambda: runner.run(h, x0, early_exit=True, threshold=0.5))
        _, loops = runner.run(h, x0, early_exit=True, threshold=0.5)
        res["mixed_exit_loops_hist"] = torch.bincount(loops.long().cpu(), minlength=7).tolist()
    log("decode exit:", res)
    return res


def run_forge_fp8(steps, warmup):
    """The Forge fp8 x fp8 GEMM (fp8_linear(quantize_input=True): e4m3
    activations and weights, v_mfma_f32_16x16x128_f8f6f4) alone on resident
    codes, timed with HIP events around the launches; 2 N K N_out flop per
    launch against the 5.0 PFLOP/s dense fp8 peak.  Also the activation
    quantization (amax + cast) on its own."""
    import torch
    from spider_moe_amd import _native as nat
    from spider_moe_amd.forge import quantize_fp8_input
    from spider_moe_amd.quant import quantize_fp8_per_tensor

    lib = nat.lib()
    out_rows = []
    for n, k, no in ((8192, 8192, 8192), (16384, 1024, 5632), (16384, 2816, 1024), (4096, 4096, 4096)):
        g = torch.Generator().manual_seed(n + k)
        x = torch.randn(n, k, generator=g).to("cuda", torch.bfloat16)
        w = (torch.randn(no, k, generator=g) / k ** 0.5).to("cuda")
        wc, ws = quantize_fp8_per_tensor(w)
        wq = wc.view(torch.uint8).contiguous()
        ws = ws.reshape(1).float().contiguous()
        xq, xs = quantize_fp8_input(x, k)
        out = torch.empty(n, no, dtype=torch.bfloat16, device="cuda")
        st = nat.stream_of(x.device)

        def gemm():
            nat.check(lib.smoe_linear_fp8fp8(xq.data_ptr(), xs.data_ptr(), n, k, wq.data_ptr(),
                                             ws.data_ptr(), None, no, 1, out.data_ptr(), nat.BF16,
                                             st), "smoe_linear_fp8fp8")

        for _ in range(warmup):
            gemm()
            quantize_fp8_input(x, k)
        torch.cuda.synchronize()
        e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        e0.record()
        for _ in range(steps):
            gemm()
        e1.record()
        for _ in range(steps):
            quantize_fp8_input(x, k)
        e2.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        qms = e1.elapsed_time(e2) / steps
        tf = 2.0 * n * k * no / (ms * 1e-3) / 1e12
        out_rows.append({"N": n, "K": k, "N_out": no, "gemm_ms": round(ms, 4),
                         "tflops": round(tf, 1), "frac_of_fp8_peak": round(tf / 5000.0, 4),
                         "quantize_ms": round(qms, 4),
                         "quantize_gbs": round(n * k * 3 / (qms * 1e-3) / 1e9, 1)})
        log("forge fp8", out_rows[-1])
        del x, w, wq, xq, out
    return out_rows


def run_quant_prefill(steps, warmup):
    """The c1 prefill block (H1024 E16 k2 m2 U2816 SwiGLU, 16384 tokens, 6
    loops) with its experts in bf16, fp8-e4m3 (per-channel scales) and int4
    (group 128, fp16 scales): ms per step and the expert GEMMs' time per
    step, each format on its own weights (the same seeded draws before
    quantization)."""
    import torch
    from spider_moe_amd import _native as nat
    from spider_moe_amd.workloads import make_block

    out = {}
    for fmt in ("bf16", "fp8", "int4"):
        wl = make_block("c1", experts=fmt, group_size=128)
        layer, h, x0 = wl.layer, wl.h, wl.x0
        with torch.no_grad():
            for _ in range(warmup):
                layer.forward_loops(h, x0)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                layer.forward_loops(h, x0)
            e1.record()
            torch.cuda.synchronize()
            timer = nat.StageTimer(stages=["up_gemm", "down_gemm"], capacity=steps * 12 + 16)
            timer.start()
            for _ in range(steps):
                layer.forward_loops(h, x0)
            st = timer.stop()
            timer.close()
        ex = layer._pack().desc.experts
        out[fmt] = {"ms_per_step": round(e0.elapsed_time(e1) / steps, 4),
                    "up_gemm_ms_per_step": round(sum(st.get("up_gemm", [0])) / steps, 4),
                    "down_gemm_ms_per_step": round(sum(st.get("down_gemm", [0])) / steps, 4),
                    "expert_weight_tiles": bool(ex.w_up_tiles),
                    "expert_weight_bytes": int(sum(t.numel() * t.element_size()
                                                   for t in layer._pack().keep
                                                   if t.dtype in (torch.uint8, torch.bfloat16)
                                                   and t.dim() == 3 and t.shape[0] == 16
                                                   and t.shape[1] in (1024, 5632)))}
        log("quant prefill", fmt, out[fmt])
        del wl, layer
        torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workloads", default="c1,c2,c3,c4")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quant-prefill", action="store_true",
                    help="only time the c1 prefill block with bf16, fp8 and int4 experts")
    ap.add_argument("--forge-fp8", action="store_true",
                    help="only time the Forge fp8 x fp8 GEMM (quantize_input=True) on four shapes")
    ap.add_argument("--decode-exit", action="store_true",
                    help="only time the c2 decode step with the early-exit gate (eager and graph)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a plain device copy of BYTES (to scale rocprof FETCH/WRITE_SIZE)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build's hot path runs on a single MI355X "
              "(multi-GPU sharding is a design note only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    if a.copy_calibration:
        src = torch.ones(a.copy_calibration, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": a.copy_calibration, "copies": 3}), flush=True)
        return
    if a.quant_prefill:
        print(json.dumps({"quant_prefill": run_quant_prefill(a.steps, a.warmup)}), flush=True)
        return
    if a.forge_fp8:
        print(json.dumps({"forge_fp8_gemm": run_forge_fp8(a.steps, a.warmup)}), flush=True)
        return
    if a.decode_exit:
        print(json.dumps({"decode_exit": run_decode_exit(a.steps, a.warmup)}), flush=True)
        return
    names = [x for x in a.workloads.split(",") if x]
    results = {nm: run_workload(nm, a.steps, a.warmup) for nm in names}
    head = results.get("c1") or results[names[0]]
    line = {
        "metric": METRIC,
        "value": head["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) hidden states, N(0,0.02) weights",
        "config": {"workload": head["desc"], "global_batch": head["tokens"], "seq_len": 1,
                   "parallelism": "none (1 GPU)", "loops": head["loops"]},
        "roofline": head["roofline"],
        "block_roofline": head["block_roofline"],
        "stage_ms_per_step": head["stage_ms_per_step"],
        "workloads": {k: v for k, v in results.items() if v is not head},
    }
    if "c2" in names:
        line["decode_exit"] = run_decode_exit(a.steps, a.warmup)
    if not a.no_cpu:
        log("cpu baseline")
        line["cpu_baseline"] = cpu_baseline(head["workload"])
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
