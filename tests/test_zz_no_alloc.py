"""smoe_block_forward_scratch (the allocation-free block forward, workspace
in a static device array) against smoe_block_forward with a caller
workspace: bit-identical outputs on two calls in a row, the second over
fewer tokens, on the fused decode front (N <= 64) and on the separate
routing stages; a workspace need above SMOE_SCRATCH_BYTES is refused."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
dev = "cuda"


def say(*a):
    print("[case]", *a, flush=True)


def _scratch_forward(layer, h, x0, loop_begin, num_loops):
    from spider_moe_amd import _native as nat
    n = h.shape[0] * h.shape[1]
    d = layer._pack().desc
    h2 = h.reshape(n, -1).contiguous()
    x2 = x0.reshape(n, -1).contiguous()
    out = torch.empty_like(h2)
    rc = nat.lib().smoe_block_forward_scratch(ctypes.byref(d), h2.data_ptr(), x2.data_ptr(),
                                              out.data_ptr(), n, loop_begin, num_loops,
                                              nat.stream_of(h2.device))
    return rc, out.view_as(h)


@pytest.mark.parametrize("case", [
    dict(name="c2", tokens=(64, 24)),                       # fp8 decode, fused front
    dict(name="c1", tokens=(200, 70), hidden_size=128, num_experts=16, expert_ffn_size=256,
         experts="bf16"),                                   # separate routing stages
], ids=["c2-front", "small-stages"])
def test_scratch_forward_matches_workspace_forward(case):
    from spider_moe_amd.workloads import make_block
    over = {k: v for k, v in case.items() if k not in ("name", "tokens")}
    n1, n2 = case["tokens"]
    for i, n in enumerate((n1, n2)):
        say("scratch forward", case["name"], "call", i, "tokens", n)
        wl = make_block(case["name"], tokens=n, seed=100 + i, **over)
        layer = wl.layer
        with torch.no_grad():
            want = layer.forward_loops(wl.h, wl.x0)
            rc, got = _scratch_forward(layer, wl.h, wl.x0, 0, layer.num_loops)
        torch.cuda.synchronize()
        assert rc == 0, rc
        assert torch.equal(got, want), (case["name"], n, float((got.float() - want.float()).abs().max()))


def test_scratch_forward_refuses_oversized_workspace():
    from spider_moe_amd import _native as nat
    from spider_moe_amd.workloads import make_block
    say("scratch forward: oversized")
    wl = make_block("c2", tokens=1024)
    layer = wl.layer
    assert layer.workspace_bytes(1024) > (8 << 20)
    rc, _ = _scratch_forward(layer, wl.h, wl.x0, 0, 1)
    torch.cuda.synchronize()
    assert rc == 3, rc  # SMOE_ECAPACITY
    assert b"static scratch" in nat.lib().smoe_last_error()


def test_scratch_forward_detects_overlap_on_another_stream():
    """The static workspace is shared: a call on a second stream while the
    first stream's call is still queued behind a bounded spin (torch's
    _sleep) is refused with SMOE_EBUSY and launches nothing; once the first
    has finished, the second stream's call runs and both equal the
    workspace forward."""
    from spider_moe_amd import _native as nat
    from spider_moe_amd.workloads import make_block
    say("scratch forward: overlap on a second stream")
    wl = make_block("c2", tokens=64)
    layer = wl.layer
    with torch.no_grad():
        want = layer.forward_loops(wl.h, wl.x0)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(sa):
        torch.cuda._sleep(100_000_000)  # ~50 ms of spinning ahead of the call on stream a
        rc_a, got_a = _scratch_forward(layer, wl.h, wl.x0, 0, layer.num_loops)
    with torch.cuda.stream(sb):
        rc_b, _ = _scratch_forward(layer, wl.h, wl.x0, 0, layer.num_loops)
    err = nat.lib().smoe_last_error()
    torch.cuda.synchronize()
    assert rc_a == 0, rc_a
    assert rc_b == 5, rc_b  # SMOE_EBUSY
    assert b"still running" in err
    with torch.cuda.stream(sb):
        rc_c, got_c = _scratch_forward(layer, wl.h, wl.x0, 0, layer.num_loops)
    torch.cuda.synchronize()
    assert rc_c == 0, rc_c
    assert torch.equal(got_a, want) and torch.equal(got_c, want)
