"""Entry points that a HIP graph can capture from a cold start.

The Q4 MoE and the no-sync pair-weighted FP8 MoE are captured in a fresh
host thread, so the first call of that thread on its stream happens inside
the capture (the library's scratch arena and stream words are created
there).  Each replay, with new inputs copied into the captured tensors and
eager work in between, equals the eager call bit for bit; for the Q4 MoE the
replays alternate between inputs whose intermediate fits fp16 and inputs
whose intermediate overflows it (the fp32 fallback), which the call's
device-side epoch must tell apart on every replay."""

from __future__ import annotations

import threading

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nat():
    from pocketlm_amd import native

    assert native.native_fp8_linear_available(), "libpocketlm_hip.so must load on the GPU box"
    return native


def _in_fresh_thread(fn):
    box = {}

    def run():
        try:
            box["value"] = fn()
        except BaseException as exc:  # re-raised in the test's thread
            box["error"] = exc

    t = threading.Thread(target=run)
    t.start()
    t.join()
    if "error" in box:
        raise box["error"]
    return box["value"]


def _q4_expert(oracle_mod, H, I, seed, gate_std, down_std):
    out = []
    for rows, cols, std, s in ((I, H, gate_std, seed), (I, H, gate_std, seed + 1), (H, I, down_std, seed + 2)):
        w = (np.random.default_rng(s).standard_normal((rows, cols)) * std).astype(np.float16).astype(np.float32)
        packed, scales, _ = oracle_mod.q4_quantize(w)
        out += [torch.from_numpy(packed).cuda(), torch.from_numpy(scales.view(np.int16)).view(torch.float16).cuda()]
    return out


def test_q4_moe_captured_cold_replays_with_and_without_fp16_overflow(nat, oracle_mod):
    H, I, S = 512, 1024, 2
    normal = [_q4_expert(oracle_mod, H, I, 300 + 3 * e, 0.02, 0.02) for e in range(S)]
    big = [_q4_expert(oracle_mod, H, I, 400 + 3 * e, 50.0, 1e-5) for e in range(S)]
    weights = [[t.clone() for t in e] for e in normal]  # the captured weight tensors
    x = torch.from_numpy(np.random.default_rng(5).standard_normal(H).astype(np.float16)).cuda()
    route = torch.tensor([0.7, 0.4], device="cuda")

    def call():
        return nat.q4_moe_selected_forward_u16(x, [tuple(e) for e in weights], route, hidden_size=H,
                                               intermediate_size=I)

    def capture():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            out = call()
        torch.cuda.synchronize()
        return graph, out

    graph, captured = _in_fresh_thread(capture)
    busy = torch.randn((256, 256), device="cuda")
    seen_overflow = False
    for trial, src in enumerate([normal, big, normal, big, big, normal]):
        for dst, s in zip(weights, src):
            for d, t in zip(dst, s):
                d.copy_(t)
        x.copy_(torch.from_numpy(np.random.default_rng(50 + trial).standard_normal(H).astype(np.float16)))
        graph.replay()
        torch.cuda.synchronize()
        eager = call()
        busy = busy @ busy.T / 256.0
        torch.cuda.synchronize()
        assert torch.equal(captured.view(torch.int16), eager.view(torch.int16)), trial
        seen_overflow = seen_overflow or src is big
    assert seen_overflow


def test_q4_moe_captured_warm_replays_with_and_without_fp16_overflow(nat, oracle_mod):
    """The capturing thread calls the Q4 MoE eagerly on its stream first, so
    its stream words exist before the capture (no zeroing inside the graph)
    and the replays rely on the epoch that the down phase advances on the
    device.  Eager calls on the same thread and stream follow the capture;
    replays alternate inputs whose intermediate fits fp16 with inputs that
    overflow it, each equal to the eager call bit for bit."""
    H, I, S = 512, 1024, 2
    normal = [_q4_expert(oracle_mod, H, I, 500 + 3 * e, 0.02, 0.02) for e in range(S)]
    big = [_q4_expert(oracle_mod, H, I, 600 + 3 * e, 50.0, 1e-5) for e in range(S)]
    weights = [[t.clone() for t in e] for e in normal]
    x = torch.from_numpy(np.random.default_rng(7).standard_normal(H).astype(np.float16)).cuda()
    route = torch.tensor([0.6, 0.5], device="cuda")

    def call():
        return nat.q4_moe_selected_forward_u16(x, [tuple(e) for e in weights], route, hidden_size=H,
                                               intermediate_size=I)

    side = torch.cuda.Stream()

    def capture():
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            first = call()  # words and arena of this (thread, stream) exist from here on
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            out = call()
        torch.cuda.synchronize()
        with torch.cuda.stream(side):
            again = call()  # an eager call on the same pair before the first replay
        torch.cuda.synchronize()
        assert torch.equal(first.view(torch.int16), again.view(torch.int16))
        return graph, out

    graph, captured = _in_fresh_thread(capture)
    seen = set()
    for trial, src in enumerate([big, normal, big, big, normal, normal, big]):
        for dst, s in zip(weights, src):
            for d, t in zip(dst, s):
                d.copy_(t)
        x.copy_(torch.from_numpy(np.random.default_rng(70 + trial).standard_normal(H).astype(np.float16)))
        graph.replay()
        torch.cuda.synchronize()
        eager = call()
        torch.cuda.synchronize()
        assert torch.equal(captured.view(torch.int16), eager.view(torch.int16)), trial
        seen.add(src is big)
    assert seen == {True, False}


def test_scratch_release_across_thread_churn(nat):
    """Each host thread keeps its own scratch arena; pocketlm_release_scratch
    frees it.  Six short-lived threads that call an entry point and release
    leave the device's free memory where it was; a thread that does not
    release keeps its arena (counted by pocketlm_scratch_bytes)."""
    from pocketlm_amd import _lib

    lib = _lib.load()
    rows, hid = 1 << 22, 16  # the top-k's logits alone take 16 MiB of scratch
    weight = (torch.randn((rows, hid), device="cuda") * 0.1).to(torch.float16)
    hidden = torch.randn((hid,), device="cuda").to(torch.float16)

    def work(release):
        def run():
            torch.cuda.set_device(0)
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                nat.lm_head_topk_u16(hidden, weight, top_k=8)
                torch.cuda.synchronize()
                held = int(lib.pocketlm_scratch_bytes())
                code = lib.pocketlm_release_scratch() if release else 0
                return held, code, int(lib.pocketlm_scratch_bytes())
        return _in_fresh_thread(run)

    work(True)  # first use: module and symbol set-up
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(6):
        held, code, after = work(True)
        assert held >= 16 << 20 and code == 0 and after == 0
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 >= free0 - (24 << 20), (free0, free1)
    held, code, after = work(False)
    assert held >= 16 << 20 and after == held


def _fp8(rows, cols, seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn((rows, cols), generator=g) * 0.02).to(torch.float8_e4m3fn).view(torch.uint8)
    s = torch.rand(((rows + 127) // 128, (cols + 127) // 128), generator=g) * 9e-3 + 1e-3
    return w.cuda(), s.cuda()


def _expert(inter, hid, seed):
    g, gs = _fp8(inter, hid, seed)
    u, us = _fp8(inter, hid, seed + 1)
    d, ds = _fp8(hid, inter, seed + 2)
    return (g, gs, u, us, d, ds)


def test_pair_weighted_nosync_captured_cold_equals_the_checked_call(nat):
    hid, inter, E, M = 512, 256, 5, 4
    items = [_expert(inter, hid, 900 + 3 * e) for e in range(E)]
    gen = torch.Generator().manual_seed(3)
    x = torch.randn((M, hid), generator=gen).to(torch.bfloat16).cuda()
    pi = torch.tensor([0, 0, 1, 2, 2, 2, 4, 3, 1], device="cuda")
    pr = torch.tensor([0, 3, 1, 0, 1, 2, 3, 3, 1], device="cuda")  # (1, 1) twice: summed in pair order
    pw = (torch.rand((9,), generator=gen) * 0.5 + 0.1).cuda()

    def capture():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            out, bad = nat.fp8_e4m3_block_mlp_many_pair_weighted_nosync(items, x, pi, pr, pw)
        torch.cuda.synchronize()
        return graph, out, bad

    graph, captured, bad = _in_fresh_thread(capture)
    for trial in range(4):
        x.copy_(torch.randn((M, hid), generator=gen).to(torch.bfloat16))
        pw.copy_(torch.rand((9,), generator=gen) * 0.5 + 0.1)
        graph.replay()
        torch.cuda.synchronize()
        want = nat.fp8_e4m3_block_mlp_many_pair_weighted_f32(items, x, pi, pr, pw)
        torch.cuda.synchronize()
        assert torch.equal(captured, want), trial
        assert int(bad.item()) == 0


def test_pair_weighted_nosync_counts_and_leaves_out_bad_pairs(nat):
    hid, inter, E, M = 256, 128, 3, 2
    items = [_expert(inter, hid, 950 + 3 * e) for e in range(E)]
    gen = torch.Generator().manual_seed(4)
    x = torch.randn((M, hid), generator=gen).cuda()
    pi = torch.tensor([0, 5, 1, 2, -1, 2], device="cuda")
    pr = torch.tensor([1, 0, 0, 7, 0, 1], device="cuda")
    pw = torch.tensor([0.5, 0.25, 0.75, 0.5, 1.0, 0.3], device="cuda")
    out, bad = nat.fp8_e4m3_block_mlp_many_pair_weighted_nosync(items, x, pi, pr, pw)
    keep = torch.tensor([0, 2, 5], device="cuda")
    want = nat.fp8_e4m3_block_mlp_many_pair_weighted_f32(items, x, pi[keep], pr[keep], pw[keep])
    torch.cuda.synchronize()
    assert int(bad.item()) == 3
    assert torch.equal(out, want)
    with pytest.raises(RuntimeError):
        nat.fp8_e4m3_block_mlp_many_pair_weighted_f32(items, x, pi, pr, pw)
