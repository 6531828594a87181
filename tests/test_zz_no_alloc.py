"""The allocation-free device-routed MoE entry point
(fp8_e4m3_block_moe_device_routed_bf16x_f32_noalloc) against the entry point
it mirrors (fp8_e4m3_block_moe_device_routed_bf16x_f32), bit for bit,
through the C ABI: two calls in a row on one device, the second smaller
than the first (the fixed scratch keeps the first call's contents), and a
call that needs more scratch than the fixed array holds.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    from pocketlm_amd import _lib

    lib = _lib.load()
    assert lib.pocketlm_device_available() == 1, "libpocketlm_hip.so must find the gfx950 device"
    return lib


def _fp8(rows, cols, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn((rows, cols), generator=g, device="cuda") * 0.02).to(torch.float8_e4m3fn).view(torch.uint8)
    s = torch.rand(((rows + 127) // 128, (cols + 127) // 128), generator=g, device="cuda") * 9e-3 + 1e-3
    return w, s


def _expert(inter, hid, seed):
    g, gs = _fp8(inter, hid, seed)
    u, us = _fp8(inter, hid, seed + 1)
    d, ds = _fp8(hid, inter, seed + 2)
    return (g, gs, u, us, d, ds)


class _Layer:
    def __init__(self, n, inter, hid, seed):
        self.n, self.inter, self.hid = n, inter, hid
        self.experts = [_expert(inter, hid, seed + 3 * e) for e in range(n)]
        self.shared = _expert(inter, hid, seed + 3 * n)
        addr = torch.tensor([[self.experts[e][r].data_ptr() for e in range(n)] for r in range(6)], dtype=torch.int64)
        self.table = addr.cuda()
        self.shared_arr = (ctypes.c_uint64 * 6)(*[t.data_ptr() for t in self.shared])


def _call(lib, fn, layer, idx, w, x, use_shared=True):
    m, k = idx.shape
    out = torch.full((m, layer.hid), float("nan"), device="cuda")
    out_s = torch.full((m, layer.hid), float("nan"), device="cuda")
    out_b = torch.zeros((m, layer.hid), dtype=torch.int16, device="cuda")
    rej = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    lib.pocketlm_set_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    code = getattr(lib, fn)(
        ctypes.c_void_p(layer.table.data_ptr()), layer.n, ctypes.c_void_p(idx.data_ptr()),
        ctypes.c_void_p(w.data_ptr()), k, ctypes.cast(layer.shared_arr, ctypes.c_void_p) if use_shared else None,
        ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()),
        ctypes.c_void_p(out_s.data_ptr()) if use_shared else None, ctypes.c_void_p(out_b.data_ptr()),
        ctypes.c_void_p(rej.data_ptr()), m, layer.inter, layer.hid, (layer.hid + 127) // 128,
        (layer.inter + 127) // 128)
    torch.cuda.synchronize()
    return code, out, out_s, out_b, rej


def _inputs(rng, m, k, n, hid, seed):
    idx = torch.from_numpy(np.stack([rng.choice(n, k, replace=False) for _ in range(m)]).astype(np.int64)).cuda()
    w = torch.from_numpy(rng.uniform(0.05, 0.5, (m, k)).astype(np.float32)).cuda()
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, hid), generator=g).to(torch.bfloat16).cuda()
    return idx, w, x


def _same(lib, layer, idx, w, x, use_shared=True):
    a = _call(lib, "fp8_e4m3_block_moe_device_routed_bf16x_f32_noalloc", layer, idx, w, x, use_shared)
    b = _call(lib, "fp8_e4m3_block_moe_device_routed_bf16x_f32", layer, idx, w, x, use_shared)
    assert a[0] == 0 and b[0] == 0
    assert torch.equal(a[1], b[1])
    if use_shared:
        assert torch.equal(a[2], b[2])
    assert torch.equal(a[3], b[3])
    assert int(a[4].item()) == int(b[4].item()) == 0
    assert torch.isfinite(a[1]).all()


def test_noalloc_equals_the_workspace_entry_point_on_two_calls(lib):
    """DeepSeek-V3 experts: four tokens of top-8 over 16 resident experts
    with the shared expert, then one token (a smaller scratch footprint in
    the same array), then one token without a shared expert."""
    layer = _Layer(16, 2048, 7168, 700)
    rng = np.random.default_rng(3)
    _same(lib, layer, *_inputs(rng, 4, 8, 16, 7168, 11))
    _same(lib, layer, *_inputs(rng, 1, 8, 16, 7168, 12))
    _same(lib, layer, *_inputs(rng, 1, 8, 16, 7168, 13), use_shared=False)


def test_noalloc_small_shapes_and_the_group_limit(lib):
    layer = _Layer(64, 256, 512, 50)
    rng = np.random.default_rng(8)
    _same(lib, layer, *_inputs(rng, 8, 8, 64, 512, 21))  # 64 routed groups + shared
    _same(lib, layer, *_inputs(rng, 2, 4, 64, 512, 22))


def test_noalloc_rejects_a_call_beyond_its_scratch(lib):
    """batch 8 x top_k 8 + shared = 65 groups of 4096 fp32 activations per
    row: 8.5 MB, over the 8 MiB array; rejected before any launch, while the
    workspace entry point runs the same call.  A following call that fits
    still matches."""
    from pocketlm_amd import _lib

    layer = _Layer(64, 4096, 256, 90)
    rng = np.random.default_rng(4)
    idx, w, x = _inputs(rng, 8, 8, 64, 256, 23)
    a = _call(lib, "fp8_e4m3_block_moe_device_routed_bf16x_f32_noalloc", layer, idx, w, x)
    assert a[0] == -2
    assert "scratch" in _lib.last_error()
    assert torch.isnan(a[1]).all()  # nothing was written
    b = _call(lib, "fp8_e4m3_block_moe_device_routed_bf16x_f32", layer, idx, w, x)
    assert b[0] == 0
    _same(lib, layer, *_inputs(rng, 2, 8, 64, 256, 24))


def test_noalloc_allocates_nothing_in_a_fresh_thread(lib):
    """After a warm-up in the main thread, a host thread that has no scratch
    yet makes several no-alloc calls through the C ABI into buffers made
    beforehand: its scratch stays at 0 bytes (a call through the workspace
    would have created an arena) and the device's free memory does not move;
    the workspace entry point then does create one, which the thread frees."""
    import threading

    layer = _Layer(16, 2048, 7168, 710)
    rng = np.random.default_rng(6)
    inputs = [_inputs(rng, m, 8, 16, 7168, 30 + m) for m in (4, 1, 2)]
    _same(lib, layer, *inputs[0])  # warm-up: module, symbols, the main thread's arena
    stream = torch.cuda.Stream()
    outs = [(torch.empty((4, 7168), device="cuda"), torch.empty((4, 7168), device="cuda"),
             torch.empty((4, 7168), dtype=torch.int16, device="cuda"), torch.empty((1,), dtype=torch.int32, device="cuda"))
            for _ in inputs]
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def call(fn, idx, w, x, o):
        m, k = idx.shape
        return getattr(lib, fn)(P(layer.table), layer.n, P(idx), P(w), k, ctypes.cast(layer.shared_arr, ctypes.c_void_p),
                                P(x), P(o[0]), P(o[1]), P(o[2]), P(o[3]), m, layer.inter, layer.hid,
                                (layer.hid + 127) // 128, (layer.inter + 127) // 128)

    # the stream's first launches set up the runtime's own per-stream memory
    lib.pocketlm_set_stream(ctypes.c_void_p(stream.cuda_stream))
    assert call("fp8_e4m3_block_moe_device_routed_bf16x_f32_noalloc", *inputs[0], outs[0]) == 0
    lib.pocketlm_set_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    box = {}

    def run():
        try:
            lib.pocketlm_set_stream(ctypes.c_void_p(stream.cuda_stream))
            free0 = torch.cuda.mem_get_info()[0]
            codes = [call("fp8_e4m3_block_moe_device_routed_bf16x_f32_noalloc", *inp, o)
                     for _ in range(3) for inp, o in zip(inputs, outs)]
            stream.synchronize()
            box["codes"] = codes
            box["free"] = (free0, torch.cuda.mem_get_info()[0])
            box["noalloc_bytes"] = int(lib.pocketlm_scratch_bytes())
            box["ws_code"] = call("fp8_e4m3_block_moe_device_routed_bf16x_f32", *inputs[0], outs[0])
            stream.synchronize()
            box["workspace_bytes"] = int(lib.pocketlm_scratch_bytes())
            box["release"] = lib.pocketlm_release_scratch()
            box["released_bytes"] = int(lib.pocketlm_scratch_bytes())
        except BaseException as exc:
            box["error"] = exc

    t = threading.Thread(target=run)
    t.start()
    t.join()
    if "error" in box:
        raise box["error"]
    assert box["codes"] == [0] * 9 and box["ws_code"] == 0
    assert box["noalloc_bytes"] == 0
    assert box["free"][0] == box["free"][1]
    assert box["workspace_bytes"] > 0 and box["release"] == 0 and box["released_bytes"] == 0
