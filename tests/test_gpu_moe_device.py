"""The device-routed MoE (fp8_e4m3_block_moe_device_routed_f32 and its bf16
twin): the router's device outputs choose the experts out of a device table.

Checked against the host-routed calls given the same experts in ascending
order (run_fp8_moe's selection, src/pcketlm/core/runtime/fp8_source.py:1600):
the weighted kernel at M = 1, the row-weighted one above, the shared expert's
MLP, bit for bit; the bf16 tail against torch's bf16 adds on the CPU
(fp8_source.py:1762, 1861-1862); left-out indices counted.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nat():
    from pocketlm_amd import native

    assert native.native_fp8_linear_available(), "libpocketlm_hip.so must load on the GPU box"
    return native


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


def _x(m, hid, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randn((m, hid), generator=g).to(torch.bfloat16).to(dtype).cuda()


def _host_routed(nat, experts, idx, w, x, shared):
    """The host-routed calls on the valid chosen experts in ascending order;
    a row that names an expert twice keeps its first weight."""
    m, k = idx.shape
    sel = sorted({int(e) for e in idx.reshape(-1) if int(e) in experts})
    route = np.zeros((len(sel), m), dtype=np.float32)
    for r in range(m):
        seen = set()
        for j in range(k):
            e = int(idx[r, j])
            if e in experts and e not in seen:
                route[sel.index(e), r] = w[r, j]
                seen.add(e)
    items = [experts[e] for e in sel]
    ys = None
    if m == 1:
        rt = torch.from_numpy(route[:, 0].copy()).cuda()
        if shared is not None:
            y, ys = nat.fp8_e4m3_block_mlp_many_weighted_shared_f32(items, shared, x, rt)
        else:
            y = nat.fp8_e4m3_block_mlp_many_weighted_f32(items, x, rt)
    else:
        y = nat.fp8_e4m3_block_mlp_many_row_weighted_f32(items, x, torch.from_numpy(route).cuda())
        if shared is not None:
            ys = nat.fp8_e4m3_block_mlp_f32(*shared, x)
    return y, ys


def _bf16_tail(y, ys):
    """torch's bf16 adds of the reference, on the CPU: zeros + routed, + shared."""
    out = torch.zeros(y.shape, dtype=torch.bfloat16) + y.cpu().to(torch.bfloat16)
    if ys is not None:
        out = out + ys.cpu().to(torch.bfloat16)
    return out


def _check(nat, table, experts, idx, w, x, shared, rejected=0):
    res = nat.fp8_e4m3_block_moe_device_routed_f32(table, x, torch.from_numpy(idx).cuda(),
                                                   torch.from_numpy(w).cuda(), shared)
    y, ys = _host_routed(nat, experts, idx, w, x, shared)
    torch.cuda.synchronize()
    assert torch.equal(res.routed, y)
    if shared is not None:
        assert torch.equal(res.shared, ys)
    else:
        assert res.shared is None
    assert torch.equal(res.output.cpu().view(torch.int16), _bf16_tail(y, ys).view(torch.int16))
    assert int(res.rejected.item()) == rejected


def _route(rng, m, k, num_experts):
    idx = np.stack([rng.choice(num_experts, k, replace=False) for _ in range(m)]).astype(np.int64)
    w = torch.from_numpy(rng.uniform(0.05, 0.5, (m, k)).astype(np.float32)).to(torch.bfloat16).float().numpy()
    return idx, w


def test_device_routed_deepseek_shapes_equal_host_routed(nat):
    """DeepSeek-V3 experts (gate/up 2048x7168, down 7168x2048): one token
    with top-8 of 12 resident experts plus the shared expert, and four tokens
    whose choices overlap."""
    experts = {e: _expert(2048, 7168, 900 + 3 * e) for e in range(12)}
    shared = _expert(2048, 7168, 990)
    table = nat.FP8ExpertTable(experts, 12)
    rng = np.random.default_rng(21)
    for m in (1, 4):
        idx, w = _route(rng, m, 8, 12)
        x = _x(m, 7168, 30 + m, torch.bfloat16)
        _check(nat, table, experts, idx, w, x, shared)


@pytest.mark.parametrize("m", [1, 2, 3, 8])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_device_routed_small_shapes_equal_host_routed(nat, m, dtype):
    hid, inter, n = 512, 256, 32
    experts = {e: _expert(inter, hid, 100 + 3 * e) for e in range(n)}
    shared = _expert(inter, hid, 99)
    table = nat.FP8ExpertTable(experts, n)
    rng = np.random.default_rng(m)
    idx, w = _route(rng, m, 4, n)
    x = _x(m, hid, 40 + m, dtype)
    _check(nat, table, experts, idx, w, x, shared)
    _check(nat, table, experts, idx, w, x, None)


def test_device_routed_at_the_group_limit(nat):
    """Eight rows of top-8 over 64 experts: 64 routed groups, the plan's
    limit, plus the shared expert as a 65th group of both launches; a row
    of all-duplicate choices keeps its first weight."""
    hid, inter, n = 512, 256, 64
    experts = {e: _expert(inter, hid, 500 + 3 * e) for e in range(n)}
    shared = _expert(inter, hid, 497)
    table = nat.FP8ExpertTable(experts, n)
    idx = np.arange(64, dtype=np.int64).reshape(8, 8)[:, ::-1].copy()  # every expert once, rows descending
    w = torch.from_numpy(np.random.default_rng(9).uniform(0.05, 0.5, (8, 8)).astype(np.float32)).to(
        torch.bfloat16).float().numpy()
    x = _x(8, hid, 60, torch.bfloat16)
    _check(nat, table, experts, idx, w, x, shared)
    idx[3] = 17  # one row names expert 17 eight times
    _check(nat, table, experts, idx, w, x, shared)


def test_device_routed_leaves_out_bad_indices(nat):
    """Indices outside [0, E) are left out and counted; an expert with a
    misaligned weight contributes nothing and is counted; a row naming an
    expert twice keeps its first weight; an id without weights contributes
    nothing."""
    hid, inter, n = 512, 256, 16
    experts = {e: _expert(inter, hid, 300 + 3 * e) for e in range(n) if e != 9}
    raw = torch.empty(inter * hid + 16, dtype=torch.uint8, device="cuda")
    raw[1:1 + inter * hid].copy_(experts[5][0].reshape(-1))
    odd = list(experts[5])
    odd[0] = raw[1:1 + inter * hid].view(inter, hid)  # 1 byte past a 16-byte boundary
    with_odd = dict(experts)
    with_odd[5] = tuple(odd)
    table = nat.FP8ExpertTable(with_odd, n)
    idx = np.array([[3, -1, 7, 3], [16, 5, 2, 11], [9, 0, 7, 200]], dtype=np.int64)
    w = np.array([[0.5, 0.25, 0.125, 0.375], [0.25, 0.5, 0.125, 0.0625], [0.5, 0.25, 0.3125, 0.125]],
                 dtype=np.float32)
    x = _x(3, hid, 50, torch.bfloat16)
    valid = {e: t for e, t in experts.items() if e != 5}
    # ids 9 (no weights) and 5 (misaligned): the host-routed reference
    # leaves them out, the device plan keeps them as empty groups, which
    # shifts the wave split of the later experts, so compare within rounding
    res = nat.fp8_e4m3_block_moe_device_routed_f32(table, x, torch.from_numpy(idx).cuda(),
                                                   torch.from_numpy(w).cuda(), None)
    y, _ys = _host_routed(nat, valid, idx, w, x, None)
    torch.cuda.synchronize()
    assert int(res.rejected.item()) == 4  # -1, 16, 200 and the misaligned expert 5
    err = (res.routed - y).norm() / y.norm()
    assert float(err) < 1e-6
    # without them the plan is the host selection exactly
    idx2 = np.where(idx == 9, 1, np.where(idx == 5, 4, idx))
    _check(nat, table, valid, idx2, w, x, None, rejected=3)


def test_device_routed_argument_errors(nat):
    hid, inter = 512, 256
    experts = {0: _expert(inter, hid, 1), 1: _expert(inter, hid, 4)}
    table = nat.FP8ExpertTable(experts, 2)
    x = _x(9, hid, 2, torch.bfloat16)
    idx = torch.zeros((9, 1), dtype=torch.int64, device="cuda")
    with pytest.raises(RuntimeError, match="code -2"):
        nat.fp8_e4m3_block_moe_device_routed_f32(table, x, idx, torch.ones((9, 1), device="cuda"))
    with pytest.raises(ValueError):
        nat.fp8_e4m3_block_moe_device_routed_f32(table, x[:, :256], idx, torch.ones((9, 1), device="cuda"))
    with pytest.raises(ValueError):
        nat.FP8ExpertTable(experts, 1)


def test_router_and_device_routed_moe_replay_in_a_hip_graph(nat):
    """The DeepSeek router and the device-routed MoE hold no host read-back,
    so the whole step captures into one HIP graph.  Each replay, with new
    router logits and hidden state copied into the captured inputs and eager
    work in between, equals the eager step."""
    hid, inter, n = 512, 256, 32
    experts = {e: _expert(inter, hid, 700 + 3 * e) for e in range(n)}
    shared = _expert(inter, hid, 697)
    table = nat.FP8ExpertTable(experts, n)
    gen = torch.Generator(device="cuda").manual_seed(13)
    logits = torch.randn((2, n), device="cuda", generator=gen)
    x = torch.randn((2, hid), device="cuda", generator=gen).to(torch.bfloat16)

    def step(lg, hx):
        idx, w = nat.route_deepseek(lg, top_k=4, n_groups=8, topk_groups=4, weights_dtype=torch.float32)
        return nat.fp8_e4m3_block_moe_device_routed_f32(table, hx, idx, w, shared)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):  # the library's workspace for this stream exists before the capture
            step(logits, x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        captured = step(logits, x)
    idx_b, w_b = nat.route_deepseek(logits, top_k=4, n_groups=8, topk_groups=4)
    idx_f, w_f = nat.route_deepseek(logits, top_k=4, n_groups=8, topk_groups=4, weights_dtype=torch.float32)
    assert torch.equal(idx_b, idx_f) and w_b.dtype == torch.bfloat16 and torch.equal(w_b.float(), w_f)
    busy = torch.randn((256, 256), device="cuda")
    for trial in range(4):
        logits.copy_(torch.randn((2, n), device="cuda", generator=gen))
        x.copy_(torch.randn((2, hid), device="cuda", generator=gen).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        eager = step(logits, x)
        busy = busy @ busy.T / 256.0  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(captured.routed, eager.routed), trial
        assert torch.equal(captured.shared, eager.shared), trial
        assert torch.equal(captured.output.view(torch.int16), eager.output.view(torch.int16)), trial
        assert int(captured.rejected.item()) == 0


def _from_logits_case(nat, table, experts, shared, logits, **kw):
    """fp8_e4m3_block_moe_from_logits equals route_deepseek followed by the
    device-routed MoE, bit for bit, indices and weights included."""
    x = kw.pop("x")
    got = nat.fp8_e4m3_block_moe_from_logits(table, x, logits, shared, **kw)
    idx, w = nat.route_deepseek(logits, weights_dtype=torch.float32, **kw)
    want = nat.fp8_e4m3_block_moe_device_routed_f32(table, x, idx, w, shared)
    torch.cuda.synchronize()
    assert torch.equal(got.indices, idx)
    assert torch.equal(got.weights, w)
    assert torch.equal(got.routed, want.routed)
    if shared is not None:
        assert torch.equal(got.shared, want.shared)
    assert torch.equal(got.output.view(torch.int16), want.output.view(torch.int16))
    assert int(got.rejected.item()) == int(want.rejected.item())
    return got


@pytest.mark.parametrize("m", [1, 3, 8])
def test_moe_from_logits_equals_router_then_device_routed(nat, m):
    """256 resident experts (hidden 512, moe_inter 256), DeepSeek-V3 routing
    (sigmoid, 8 groups keep 4, top 8, x2.5) with and without a correction
    bias, softmax scoring, and flat top-8."""
    hid, inter, n = 512, 256, 256
    experts = {e: _expert(inter, hid, 3000 + 3 * e) for e in range(n)}
    shared = _expert(inter, hid, 2999)
    table = nat.FP8ExpertTable(experts, n)
    g = torch.Generator().manual_seed(40 + m)
    logits = torch.randn((m, n), generator=g).cuda()
    x = _x(m, hid, 50 + m, torch.bfloat16)
    bias = (torch.randn((n,), generator=g) * 0.1).cuda()
    _from_logits_case(nat, table, experts, shared, logits, x=x)
    _from_logits_case(nat, table, experts, shared, logits, x=x, bias=bias)
    _from_logits_case(nat, table, experts, None, logits, x=x, scoring_func="softmax", top_k=4)
    _from_logits_case(nat, table, experts, shared, logits, x=x, n_groups=1, topk_groups=1)


def test_moe_from_logits_deepseek_shapes_and_nan_logits(nat):
    """DeepSeek-V3 experts over 16 resident slots (2 per group); a NaN logit
    sends that row through the rounds path of the router; the batch of two
    and each of its rows alone."""
    experts = {e: _expert(2048, 7168, 4000 + 3 * e) for e in range(16)}
    shared = _expert(2048, 7168, 3990)
    table = nat.FP8ExpertTable(experts, 16)
    g = torch.Generator().manual_seed(77)
    logits = torch.randn((2, 16), generator=g)
    logits[1, 5] = float("nan")
    x = _x(2, 7168, 78, torch.bfloat16)
    _from_logits_case(nat, table, experts, shared, logits.cuda(), x=x)
    _from_logits_case(nat, table, experts, shared, logits[1:].cuda(), x=x[1:].contiguous())
    _from_logits_case(nat, table, experts, shared, logits[:1].cuda(), x=x[:1].contiguous())


def test_moe_from_logits_one_row_deepseek_shapes_and_graph_replays(nat):
    """The decode step's case: one row, 256 experts (ids over 8 weight sets
    of the DeepSeek-V3 shapes, 2048 x 7168), the shared expert and a
    correction bias.  Eager calls with new logits each time, then a HIP
    graph replayed with new logits and eager work in between: every result
    equals route_deepseek followed by the device-routed call, bit for bit."""
    sets = [_expert(2048, 7168, 6000 + 3 * i) for i in range(8)]
    experts = {e: sets[e % 8] for e in range(256)}
    shared = _expert(2048, 7168, 5990)
    table = nat.FP8ExpertTable(experts, 256)
    g = torch.Generator().manual_seed(91)
    bias = (torch.randn((256,), generator=g) * 0.1).cuda()
    x = _x(1, 7168, 92, torch.bfloat16)
    for _ in range(3):
        _from_logits_case(nat, table, experts, shared, torch.randn((1, 256), generator=g).cuda(), x=x, bias=bias)
    _from_logits_case(nat, table, experts, None, torch.randn((1, 256), generator=g).cuda(), x=x)

    logits = torch.randn((1, 256), generator=g).cuda()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            nat.fp8_e4m3_block_moe_from_logits(table, x, logits, shared, bias=bias)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        captured = nat.fp8_e4m3_block_moe_from_logits(table, x, logits, shared, bias=bias)
    busy = torch.randn((256, 256), device="cuda")
    for trial in range(4):
        logits.copy_(torch.randn((1, 256), generator=g).cuda())
        graph.replay()
        torch.cuda.synchronize()
        idx, w = nat.route_deepseek(logits, weights_dtype=torch.float32, bias=bias)
        want = nat.fp8_e4m3_block_moe_device_routed_f32(table, x, idx, w, shared)
        busy = busy @ busy.T / 256.0  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(captured.indices, idx), trial
        assert torch.equal(captured.weights, w), trial
        assert torch.equal(captured.routed, want.routed), trial
        assert torch.equal(captured.shared, want.shared), trial
        assert torch.equal(captured.output.view(torch.int16), want.output.view(torch.int16)), trial


@pytest.mark.parametrize("n,resident", [(384, 48), (2048, 16)])
def test_moe_from_logits_wide_tables(nat, n, resident):
    """Tables wider than 256 experts (no table copy in LDS; 16 and 64 experts
    per router lane), most ids without weights (null addresses: those picks
    contribute nothing), batches of 1 and 6 rows."""
    hid, inter = 256, 128
    experts = {e: _expert(inter, hid, 5000 + 3 * e) for e in range(0, n, n // resident)}
    table = nat.FP8ExpertTable(experts, n)
    g = torch.Generator().manual_seed(n)
    for m in (1, 6):
        logits = torch.randn((m, n), generator=g).cuda()
        x = _x(m, hid, 60 + m, torch.bfloat16)
        _from_logits_case(nat, table, experts, None, logits, x=x)
