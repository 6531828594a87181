"""FP8 weights in 8-row tiles: the pack against an independent torch
restatement of the layout (bit-exact), the tiles8 linears against the
row-major linears (bit-exact: same kernel and arithmetic, other weight
addresses) and against the oracle (rel-L2 1e-5), and the error codes.
The packed format has no counterpart in the reference."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import rel_l2

TOL = 1e-5


def synth_fp8(rows, cols, seed, std=0.02):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn((rows, cols), generator=g) * std).to(torch.float8_e4m3fn).view(torch.uint8)
    s = (torch.rand(((rows + 127) // 128, (cols + 127) // 128), generator=g) * 9e-3 + 1e-3).float()
    return w, s


def synth_x(m, k, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn((m, k), generator=g).to(torch.bfloat16)


def tiles_by_reshape(w: torch.Tensor) -> torch.Tensor:
    """The layout restated with torch: pad to whole 8 x 128 tiles, then
    [tile row][row][block][col] -> [tile row][block][row][col]."""
    rows, cols = w.shape
    r8, nb = -(-rows // 8), -(-cols // 128)
    p = torch.zeros((r8 * 8, nb * 128), dtype=torch.uint8, device=w.device)
    p[:rows, :cols] = w
    return p.reshape(r8, 8, nb, 128).permute(0, 2, 1, 3).contiguous().reshape(-1)


def test_tiles8_bytes_on_the_host():
    from pocketlm_amd import _lib

    lib = _lib.load()
    assert lib.fp8_e4m3_tiles8_bytes(7168, 16384) == 7168 * 16384
    assert lib.fp8_e4m3_tiles8_bytes(37, 2000) == 5 * 16 * 1024
    assert lib.fp8_e4m3_tiles8_bytes(1, 1) == 1024
    assert lib.fp8_e4m3_tiles8_bytes(0, 128) == -2
    assert lib.fp8_e4m3_tiles8_bytes(128, -1) == -2


@pytest.fixture(scope="module")
def nat():
    from pocketlm_amd import native

    assert native.native_fp8_linear_available(), "libpocketlm_hip.so must load on the GPU box"
    return native


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols", [(37, 2000), (8, 128), (300, 7168), (129, 2003), (7168, 16384)])
def test_pack_matches_the_layout(nat, rows, cols):
    print(f"pack tiles8 {rows}x{cols}", flush=True)
    w, _ = synth_fp8(rows, cols, rows + cols)
    wd = w.cuda()
    if cols % 16:
        # an unaligned source row start: the byte path
        wd = torch.empty(rows * cols + 1, dtype=torch.uint8, device="cuda")[1:].view(rows, cols)
        wd.copy_(w.cuda())
    packed = nat.pack_fp8_tiles8(wd)
    torch.cuda.synchronize()
    assert packed.tiles.numel() == -(-rows // 8) * -(-cols // 128) * 1024
    assert torch.equal(packed.tiles, tiles_by_reshape(w.cuda()))


@pytest.mark.gpu
@pytest.mark.parametrize(
    "rows,cols,ms",
    [
        (7168, 16384, (1, 2, 8)),   # o projection: 1-tile waves at one row, 4-tile waves at 8
        (24576, 1536, (1, 3)),      # q_b: 4-tile waves at one row
        (576, 7168, (1, 8)),        # kv_a: 8-deep pipeline
        (37, 2000, (1, 2, 5, 8)),   # ragged rows and a ragged last block
        (300, 7168, (9,)),          # two launches of the batch
    ],
)
def test_tiles8_linear_equals_the_row_major_linear(nat, oracle_mod, rows, cols, ms):
    w, s = synth_fp8(rows, cols, 3 * rows + cols)
    wd, sd = w.cuda(), s.cuda()
    packed = nat.pack_fp8_tiles8(wd)
    for m in ms:
        print(f"tiles8 linear {rows}x{cols} m={m}", flush=True)
        xb = synth_x(m, cols, m + rows).cuda()
        for x in (xb, xb.float()):
            want = nat.fp8_e4m3_block_linear_f32(wd, sd, x)
            got = nat.fp8_e4m3_block_linear_tiles8_f32(packed, sd, x)
            torch.cuda.synchronize()
            assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (m, x.dtype)
        if rows * cols <= 2_200_000:
            ref = oracle_mod.fp8_linear(w.numpy(), s.numpy(), xb.float().cpu().numpy())
            assert rel_l2(got.cpu().numpy(), ref) < TOL


@pytest.mark.gpu
def test_tiles8_linear_nan_bytes_redo(nat):
    # e4m3 NaN bytes add nothing, as in the row-major linear (its NaN redo pass)
    w, s = synth_fp8(256, 2048, 9)
    w[7, 100] = 0x7F
    w[40, 1500] = 0xFF
    w[200, :16] = 0x7F
    wd, sd = w.cuda(), s.cuda()
    x = synth_x(3, 2048, 10).cuda()
    got = nat.fp8_e4m3_block_linear_tiles8_f32(nat.pack_fp8_tiles8(wd), sd, x)
    want = nat.fp8_e4m3_block_linear_f32(wd, sd, x)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


@pytest.mark.gpu
def test_tiles8_error_codes(nat):
    from pocketlm_amd import _lib

    lib = _lib.load()
    w, s = synth_fp8(64, 2008, 1)
    wd, sd = w.cuda(), s.cuda()
    tiles = torch.empty(lib.fp8_e4m3_tiles8_bytes(64, 2008) + 16, dtype=torch.uint8, device="cuda")
    x = torch.zeros((1, 2008), dtype=torch.float32, device="cuda")
    y = torch.empty((1, 64), dtype=torch.float32, device="cuda")
    p = ctypes.c_void_p
    assert lib.fp8_e4m3_pack_tiles8(None, p(tiles.data_ptr()), 64, 2008) == -1
    assert lib.fp8_e4m3_pack_tiles8(p(wd.data_ptr()), p(tiles.data_ptr() + 8), 64, 2008) == -2
    assert lib.fp8_e4m3_pack_tiles8(p(wd.data_ptr()), p(tiles.data_ptr()), 0, 2008) == -2
    assert lib.fp8_e4m3_pack_tiles8(p(wd.data_ptr()), p(tiles.data_ptr()), 64, 2008) == 0
    # in_cols % 16 != 0 has no tiles8 path
    assert lib.fp8_e4m3_block_linear_tiles8_f32(p(tiles.data_ptr()), p(sd.data_ptr()), p(x.data_ptr()),
                                                p(y.data_ptr()), 1, 64, 2008, 16) == -2
    assert lib.fp8_e4m3_block_linear_tiles8_f32(None, p(sd.data_ptr()), p(x.data_ptr()), p(y.data_ptr()),
                                                1, 64, 2008, 16) == -1
    torch.cuda.synchronize()
