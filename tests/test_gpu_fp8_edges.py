"""Edge paths of the matrix-core FP8 kernels against the oracle.

* K that is a multiple of 16 but not of 128: the last block of every row is
  partial (the linear family's pipelined loop masks it; the gate/up and down
  phases skip its missing columns).
* fp32 activations that are not bf16 values (the hi + lo split of the B
  operand), next to the bf16 twins.
* NaN weight bytes in the gate, up and down matrices of a MoE: the NaN redo
  pass of both kernels must give the oracle's values (NaN bytes count as 0,
  fp8_linear.cpp:31-33).
* An infinite activation: the redo pass splits it exactly, so every output
  row is +-inf (or NaN where a weight byte of that column is 0), as the
  oracle's sequential sums give.
* Batches above 8 rows through the MLP (launches of 8 rows at offsets).

Bars: rel-L2 1e-5 against the oracle; batched calls bit-exact to one-row
calls (torch.equal).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-5


@pytest.fixture(scope="module")
def nat():
    from pocketlm_amd import native

    assert native.native_fp8_linear_available(), "libpocketlm_hip.so must load on the GPU box"
    return native


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def synth_fp8(rows, cols, seed, std=0.02):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn((rows, cols), generator=g) * std).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    s = (torch.rand(((rows + 127) // 128, (cols + 127) // 128), generator=g) * 9e-3 + 1e-3).numpy().astype(np.float32)
    return w, s


def fp32_x(m, k, seed):
    """Full-precision fp32 activations (not bf16 values)."""
    return np.random.default_rng(seed).standard_normal((m, k)).astype(np.float32)


def rows_of(fn, x):
    return torch.cat([fn(x[i:i + 1]) for i in range(x.shape[0])])


@pytest.mark.parametrize("n,k", [(72, 144), (200, 400), (136, 1040), (264, 2064)])
def test_ragged_k_linear_and_dual(nat, oracle_mod, n, k):
    print("ragged linear", n, k, flush=True)
    w, s = synth_fp8(n, k, 7000 + k)
    w2, s2 = synth_fp8(n, k, 7100 + k)
    x = fp32_x(5, k, k)
    dw, ds, dx = dev(w), dev(s), dev(x)
    y = nat.fp8_e4m3_block_linear_f32(dw, ds, dx)
    assert rel_l2(host(y), oracle_mod.fp8_linear(w, s, x)) < TOL
    assert torch.equal(y, rows_of(lambda xi: nat.fp8_e4m3_block_linear_f32(dw, ds, xi), dx))
    ya, yb = nat.fp8_e4m3_block_dual_linear_f32(dw, ds, dev(w2), dev(s2), dx)
    assert torch.equal(ya, y)
    assert torch.equal(yb, nat.fp8_e4m3_block_linear_f32(dev(w2), dev(s2), dx))
    # bf16 activations: the twin equals the fp32 call on the widened values
    xb = dx.to(torch.bfloat16)
    assert torch.equal(nat.fp8_e4m3_block_linear_f32(dw, ds, xb), nat.fp8_e4m3_block_linear_f32(dw, ds, xb.float()))


@pytest.mark.parametrize("inter,hid", [(144, 400), (272, 528)])
def test_ragged_k_mlp(nat, oracle_mod, inter, hid):
    print("ragged mlp", inter, hid, flush=True)
    g, gs = synth_fp8(inter, hid, 11 + hid)
    u, us = synth_fp8(inter, hid, 12 + hid)
    d, ds = synth_fp8(hid, inter, 13 + hid)
    x = fp32_x(3, hid, inter)
    args = [dev(a) for a in (g, gs, u, us, d, ds)]
    y = nat.fp8_e4m3_block_mlp_f32(*args, dev(x))
    assert rel_l2(host(y), oracle_mod.fp8_mlp(g, gs, u, us, d, ds, x)) < TOL
    assert torch.equal(y, rows_of(lambda xi: nat.fp8_e4m3_block_mlp_f32(*args, xi), dev(x)))


def test_mlp_batch_above_eight_rows(nat, oracle_mod):
    g, gs = synth_fp8(256, 512, 41)
    u, us = synth_fp8(256, 512, 42)
    d, ds = synth_fp8(512, 256, 43)
    x = fp32_x(11, 512, 44)
    args = [dev(a) for a in (g, gs, u, us, d, ds)]
    y = nat.fp8_e4m3_block_mlp_f32(*args, dev(x))
    assert rel_l2(host(y), oracle_mod.fp8_mlp(g, gs, u, us, d, ds, x)) < TOL
    assert torch.equal(y[9:10], nat.fp8_e4m3_block_mlp_f32(*args, dev(x[9:10])))


def _moe_items(n_exp, inter, hid, seed):
    items = []
    for e in range(n_exp):
        g, gs = synth_fp8(inter, hid, seed + 3 * e)
        u, us = synth_fp8(inter, hid, seed + 3 * e + 1)
        d, ds = synth_fp8(hid, inter, seed + 3 * e + 2)
        items.append([g, gs, u, us, d, ds])
    return items


def test_nan_bytes_in_moe_experts(nat, oracle_mod):
    items = _moe_items(4, 256, 512, 900)
    items[0][0][5, 17] = 0x7F      # gate of expert 0
    items[1][2][100, 300:316] = 0xFF  # up of expert 1, a whole 16-byte piece
    items[2][4][33, 200] = 0x7F    # down of expert 2
    items[3][4][511, 255] = 0xFF   # down of expert 3, last row and column
    items = [tuple(it) for it in items]
    di = [tuple(dev(a) for a in it) for it in items]
    x = fp32_x(3, 512, 901)
    route = np.array([0.4, 0.3, 0.2, 0.1], dtype=np.float32)
    y = nat.fp8_e4m3_block_mlp_many_weighted_f32(di, dev(x[:1]), dev(route))
    assert np.isfinite(host(y)).all()
    assert rel_l2(host(y), oracle_mod.fp8_mlp_many_weighted(items, x[:1], route)) < TOL
    rroute = np.array([[0.5, 0.0, 0.2], [0.1, 0.3, 0.0], [0.0, 0.2, 0.6], [0.4, 0.5, 0.2]], dtype=np.float32)
    yr = nat.fp8_e4m3_block_mlp_many_row_weighted_f32(di, dev(x), dev(rroute))
    assert np.isfinite(host(yr)).all()
    assert rel_l2(host(yr), oracle_mod.fp8_mlp_many_row_weighted(items, x, rroute)) < TOL
    one = nat.fp8_e4m3_block_mlp_many_row_weighted_f32(di, dev(x[1:2]), dev(np.ascontiguousarray(rroute[:, 1:2])))
    assert torch.equal(yr[1:2], one)


def test_infinite_activation(nat, oracle_mod):
    w, s = synth_fp8(192, 512, 77)
    x = fp32_x(2, 512, 78)
    x[0, 130] = np.inf
    x[1, 5] = -np.inf
    y = host(nat.fp8_e4m3_block_linear_f32(dev(w), dev(s), dev(x)))
    want = oracle_mod.fp8_linear(w, s, x)
    assert np.array_equal(np.isnan(y), np.isnan(want))
    assert np.array_equal(y[np.isinf(want)], want[np.isinf(want)])
    fin = np.isfinite(want)
    assert np.isinf(want).any() and np.array_equal(np.isfinite(y), fin)
