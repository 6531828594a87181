"""The DeepSeek MoE layer orchestration (run_fp8_moe,
src/pcketlm/core/runtime/fp8_source.py:1569-1884): the oracle's restatement
pinned on the CPU, the device module checked against it on the GPU."""

from __future__ import annotations

import numpy as np
import pytest
import torch

H, I, E, TOPK = 512, 256, 32, 4


def _fp8(rng, shape):
    w = torch.from_numpy((rng.standard_normal(shape) * 0.02).astype(np.float32))
    return w.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _expert(rng):
    gs = (rng.random((I // 128, H // 128)) * 9e-3 + 1e-3).astype(np.float32)
    us = (rng.random((I // 128, H // 128)) * 9e-3 + 1e-3).astype(np.float32)
    ds = (rng.random((H // 128, I // 128)) * 9e-3 + 1e-3).astype(np.float32)
    return (_fp8(rng, (I, H)), gs, _fp8(rng, (I, H)), us, _fp8(rng, (H, I)), ds)


def _layer(seed, m, oracle_mod):
    rng = np.random.default_rng(seed)
    experts = {e: _expert(rng) for e in range(E)}
    shared = _expert(rng)
    x = torch.from_numpy(rng.standard_normal((m, H)).astype(np.float32)).to(torch.bfloat16).float().numpy()
    logits = rng.standard_normal((m, E)).astype(np.float32)
    idx, w = oracle_mod.deepseek_route(logits, top_k=TOPK, n_groups=8, topk_groups=4)
    return experts, shared, x, idx, w


def _fp64_layer(oracle_mod, experts, shared, x, idx, w):
    """Closed form: sum over the row's selected experts of route * SwiGLU MLP, plus the shared MLP."""
    def mlp(ex, v):
        g, gs, u, us, d, ds = ex
        deq = lambda q, s: oracle_mod.fp8_dequant(q, s, "f32").astype(np.float64)
        a = deq(g, gs) @ v
        b = deq(u, us) @ v
        h = a / (1.0 + np.exp(-a)) * b
        return deq(d, ds) @ h
    out = np.zeros_like(x, dtype=np.float64)
    for r in range(x.shape[0]):
        for e, wt in zip(idx[r], w[r]):
            out[r] += float(wt) * mlp(experts[int(e)], x[r].astype(np.float64))
        out[r] += mlp(shared, x[r].astype(np.float64))
    return out


def test_oracle_moe_layer_paths_pinned(oracle_mod):
    experts, shared, x, idx, w = _layer(5, 3, oracle_mod)
    want = _fp64_layer(oracle_mod, experts, shared, x, idx, w)
    outs = {}
    for mode in ("auto", "row", "pair"):
        y, sel, path = oracle_mod.run_fp8_moe(x, idx, w, experts, shared, mode=mode)
        assert sel == sorted(set(idx.reshape(-1).tolist()))
        outs[path] = y
        # bf16 output: within a few bf16 roundings of the fp64 layer
        assert np.abs(y - want).max() < 2e-2 * np.abs(want).max(), path
    assert set(outs) == {"per_expert", "row_weighted", "pair_weighted"}
    # pair-weighted == row-weighted bit for bit (test_native_fp8_linear.py:202-247)
    assert np.array_equal(outs["row_weighted"], outs["pair_weighted"])
    # one row alone takes the weighted path and agrees with the batched paths
    y1, _sel, path1 = oracle_mod.run_fp8_moe(x[1:2], idx[1:2], w[1:2], experts, shared)
    assert path1 == "weighted"
    assert np.abs(y1[0] - outs["row_weighted"][1]).max() <= 2 ** -7 * np.abs(y1[0]).max() + 1e-6
    # a planted mistake (route weights dropped) must fail the closed form
    bad, _s, _p = oracle_mod.run_fp8_moe(x, idx, np.ones_like(w), experts, shared)
    assert np.abs(bad - want).max() > 5e-2 * np.abs(want).max()


@pytest.mark.gpu
@pytest.mark.parametrize("m,env", [(1, None), (3, None), (3, "PCKETLM_ENABLE_FP8_MOE_ROW_WEIGHTED_MANY"),
                                   (3, "PCKETLM_ENABLE_FP8_MOE_PAIR_WEIGHTED_MANY")])
def test_device_moe_layer_vs_oracle(oracle_mod, monkeypatch, m, env):
    from pocketlm_amd import moe

    if env:
        monkeypatch.setenv(env, "1")
    experts, shared, x, idx, w = _layer(11 + m, m, oracle_mod)
    mode = {None: "auto", "PCKETLM_ENABLE_FP8_MOE_ROW_WEIGHTED_MANY": "row",
            "PCKETLM_ENABLE_FP8_MOE_PAIR_WEIGHTED_MANY": "pair"}[env]
    want, sel, path = oracle_mod.run_fp8_moe(x, idx, w, experts, shared, mode=mode)
    dev_experts = {e: tuple(torch.from_numpy(t).cuda() for t in ex) for e, ex in experts.items()}
    dev_shared = tuple(torch.from_numpy(t).cuda() for t in shared)
    res = moe.run_fp8_moe(torch.from_numpy(x).cuda().to(torch.bfloat16), torch.from_numpy(idx).cuda(),
                          torch.from_numpy(w).cuda().to(torch.bfloat16), dev_experts, dev_shared)
    torch.cuda.synchronize()
    got = res.output.float().cpu().numpy()
    assert res.selected_experts == sel and res.path == path
    assert res.output.dtype == torch.bfloat16 and tuple(res.output.shape) == (m, H)
    # fp32 results agree to ~1e-7 before the bf16 roundings: at most one bf16
    # step apart, and almost all elements identical.
    diff = np.abs(got - want)
    assert (diff <= np.abs(want) * 2 ** -7 + 1e-7).all()
    assert (diff == 0).mean() > 0.97


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 3])
def test_device_routed_layer_equals_host_routed_layer(oracle_mod, monkeypatch, m):
    """run_fp8_moe_device (experts chosen on the device, bf16 tail in the
    library) gives run_fp8_moe's bf16 output bit for bit: the weighted path
    at M = 1, the row-weighted path at M = 3; and the oracle's layer within
    one bf16 step."""
    from pocketlm_amd import moe, native

    monkeypatch.setenv("PCKETLM_ENABLE_FP8_MOE_ROW_WEIGHTED_MANY", "1")
    experts, shared, x, idx, w = _layer(31 + m, m, oracle_mod)
    dev_experts = {e: tuple(torch.from_numpy(t).cuda() for t in ex) for e, ex in experts.items()}
    dev_shared = tuple(torch.from_numpy(t).cuda() for t in shared)
    table = native.FP8ExpertTable(dev_experts, E)
    xd = torch.from_numpy(x).cuda().to(torch.bfloat16)
    idx_d = torch.from_numpy(idx).cuda()
    w_d = torch.from_numpy(w).cuda().to(torch.bfloat16)
    got = moe.run_fp8_moe_device(xd, idx_d, w_d, table, dev_shared)
    ref = moe.run_fp8_moe(xd, idx_d, w_d, dev_experts, dev_shared)
    torch.cuda.synchronize()
    assert got.path == "device_routed" and ref.path == ("weighted" if m == 1 else "row_weighted")
    assert got.output.dtype == torch.bfloat16 and tuple(got.output.shape) == (m, H)
    assert torch.equal(got.output.view(torch.int16), ref.output.view(torch.int16))
    want, _sel, _path = oracle_mod.run_fp8_moe(x, idx, w, experts, shared, mode="auto" if m == 1 else "row")
    diff = np.abs(got.output.float().cpu().numpy() - want)
    assert (diff <= np.abs(want) * 2 ** -7 + 1e-7).all()
