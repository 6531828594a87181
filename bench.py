#!/usr/bin/env python3
"""Benchmark of the quantized-decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]      # one JSON line
    python bench.py --table [--table-out FILE]               # every workload

Default line: one decode token through a DeepSeek-V3 MoE layer (hidden 7168,
256 routed experts + 1 shared expert, moe_inter 2048, SwiGLU; every expert's
gate/up [2048, 7168] and down [7168, 2048] FP8 e4m3 from N(0, 0.02) with
fp32 128x128-block scale_inv ~U(1e-3, 1e-2)).  All 257 experts (11.3 GB) are
resident in HBM, so the 256 MB Infinity Cache cannot serve the chosen ones.
One step = one token (M = 1, a bf16 hidden state ~N(0, 1)) as the device
path runs it:

fp8_e4m3_block_moe_from_logits_bf16x_f32 on fresh router logits ~N(0, 1),
three launches:

  1. routing (sigmoid scores, 8 groups of which the best 4 are kept, group
     score = max: no correction bias, top 8, normalised, x2.5; the choices
     of ds_route_topk_f32) and the plan of the chosen experts;
  2. gate/up + SiLU for the 8 chosen experts and the shared expert;
  3. down + route-weighted sum + the shared expert + the bf16 output.

The roofline is taken over the MoE layer's own launches (plan, gate/up,
down): fp8_e4m3_block_moe_device_routed_bf16x_f32 on the router outputs the
timed steps wrote, timed in a separate region.  The same steps as two calls
(ds_route_topk_f32, then the device-routed MoE) are timed too.  The line also carries "m8": the speculative / MTP
verifier batch, M = 8 bf16 activation rows, on the 7168 x 16384 output
projection (each weight byte read once per batch), and "verifier": every
DeepSeek-V3 projection shape of that batch at M = 1 and M = 8.

Timing: the stream is held by a short sleep kernel while the timed launches
are queued; one HIP event pair on the launch stream brackets all of them, and
the GPU runs them back to back.

cpu_baseline: the reference's own fp8_linear.cpp, compiled from its source
into oracle/_ref (fp8_e4m3_block_mlp_many_weighted_f32 for the 8 routed
experts + fp8_e4m3_block_mlp_f32 for the shared expert, as run_fp8_moe calls
them at M = 1), on the host's cores and on one thread, on a bounded sample.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import subprocess
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
PEAK_HBM_GBS = 8000.0
MALL_BYTES = 1 << 30  # rotate at least this many distinct weight bytes

# DeepSeek-V3 MoE layer
HID, INTER, N_ROUTED, TOP_K = 7168, 2048, 256, 8
N_GROUPS, TOPK_GROUPS, ROUTE_SCALE = 8, 4, 2.5


def _args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--table", action="store_true", help="measure every workload, print a markdown table")
    ap.add_argument("--table-out", default=None, help="also write the table to this file")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample length (all threads)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default=None,
                    help="table: measure only the workloads whose name contains one of these comma-separated "
                         "strings (for profiling one workload)")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="run a few default steps, then a plain 256 MiB device copy, for counter runs "
                         "(rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE); prints nothing else")
    return ap.parse_args(argv)


# --------------------------------------------------------------------------- timing

class Timer:
    """GPU time of a batch of launches from one pair of HIP events on the
    launch stream.  The launches are queued behind a sleep kernel first, so
    the host's enqueue cost stays out of the timed region and the kernels run
    back to back."""

    def __init__(self, torch):
        self.torch = torch
        self.cycles_per_ms = self._calibrate()

    def _calibrate(self) -> float:
        torch = self.torch
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        torch.cuda._sleep(2_000_000)
        b.record()
        torch.cuda.synchronize()
        ms = max(a.elapsed_time(b), 1e-3)
        return 2_000_000 / ms

    def run(self, launches, hold_ms: float | None = None) -> float:
        """launches: zero-arg callables, each enqueuing kernels on the current
        stream.  Returns the total GPU time of all of them in ms."""
        torch = self.torch
        if hold_ms is None:
            hold_ms = max(30.0, 0.1 * len(launches))
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        torch.cuda._sleep(int(self.cycles_per_ms * hold_ms))
        start.record()
        for fn in launches:
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end)


def _stream_ptr(torch):
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _vp(t):
    return ctypes.c_void_p(t.data_ptr())


# --------------------------------------------------------------------------- byte counts

def fp8_bytes(rows, cols, m):
    """FP8 GEMV: weights, fp32 scale grid, bf16 activations, fp32 outputs."""
    return rows * cols + 4 * math.ceil(rows / 128) * math.ceil(cols / 128) + 2 * m * cols + 4 * m * rows


def expert_bytes(hidden=HID, inter=INTER):
    """One SwiGLU expert at rest: gate, up [inter, hidden] and down
    [hidden, inter] e4m3 bytes and their fp32 scale grids."""
    grid_gu = math.ceil(inter / 128) * math.ceil(hidden / 128)
    grid_d = math.ceil(hidden / 128) * math.ceil(inter / 128)
    return 3 * inter * hidden + 4 * (2 * grid_gu + grid_d)


def moe_layer_bytes(m=1):
    """One MoE layer step: the 8 chosen + the shared expert at rest, the
    bf16 hidden rows in, the fp32 layer output rows out."""
    return (TOP_K + 1) * expert_bytes() + 2 * m * HID + 4 * m * HID


def moe_step_bytes(m=1):
    """... plus the router logits read by the routing launch."""
    return moe_layer_bytes(m) + 4 * m * N_ROUTED


# --------------------------------------------------------------------------- DeepSeek-V3 MoE layer

class MoEPool:
    """The 256 routed experts and the shared expert of one DeepSeek-V3 MoE
    layer in HBM, the device table of the routed experts' addresses
    ([6][256] int64: gate w/s, up w/s, down w/s) and the shared expert's."""

    def __init__(self, torch, seed=20261201):
        self.torch = torch
        gen = torch.Generator(device="cuda").manual_seed(seed)
        self.experts = []
        for _ in range(N_ROUTED + 1):
            t = []
            for rows, cols in ((INTER, HID), (INTER, HID), (HID, INTER)):
                w = torch.randn((rows, cols), generator=gen, device="cuda").mul_(0.02)
                t.append(w.to(torch.float8_e4m3fn).view(torch.uint8))
                del w
                t.append(torch.rand((math.ceil(rows / 128), math.ceil(cols / 128)), generator=gen,
                                    device="cuda").mul_(9e-3).add_(1e-3))
            self.experts.append(t)
        addr = torch.tensor([[self.experts[e][r].data_ptr() for e in range(N_ROUTED)] for r in range(6)],
                            dtype=torch.int64)
        self.table = addr.cuda()
        self.shared = (ctypes.c_uint64 * 6)(*[t.data_ptr() for t in self.experts[N_ROUTED]])
        torch.cuda.synchronize()

    def nbytes(self):
        return sum(t.numel() * t.element_size() for e in self.experts for t in e)


class MoEStep:
    """One decode token through the layer, as the device path runs it."""

    def __init__(self, torch, lib, pool, nsteps, seed=7):
        self.torch, self.lib, self.pool = torch, lib, pool
        gen = torch.Generator(device="cuda").manual_seed(seed)
        self.nsteps = nsteps
        self.logits = torch.randn((nsteps, N_ROUTED), generator=gen, device="cuda")
        self.x = torch.randn((nsteps, HID), generator=gen, device="cuda").to(torch.bfloat16)
        self.idx = torch.empty((nsteps, TOP_K), dtype=torch.int64, device="cuda")
        self.w = torch.empty((nsteps, TOP_K), dtype=torch.float32, device="cuda")
        self.y = torch.empty((1, HID), device="cuda")
        self.ys = torch.empty((1, HID), device="cuda")
        self.ybf = torch.empty((1, HID), dtype=torch.bfloat16, device="cuda")
        self.rejected = torch.zeros((1,), dtype=torch.int32, device="cuda")
        self.row_bytes = {"logits": 4 * N_ROUTED, "x": 2 * HID, "idx": 8 * TOP_K, "w": 4 * TOP_K}

    def _at(self, t, i, name):
        return ctypes.c_void_p(t.data_ptr() + i * self.row_bytes[name])

    def route(self, i):
        code = self.lib.ds_route_topk_f32(self._at(self.logits, i, "logits"), None, 1, N_ROUTED, TOP_K, N_GROUPS,
                                          TOPK_GROUPS, 0, ROUTE_SCALE, self._at(self.idx, i, "idx"),
                                          self._at(self.w, i, "w"))
        if code != 0:
            raise RuntimeError(f"ds_route_topk_f32 failed with code {code}")

    def moe(self, i):
        code = self.lib.fp8_e4m3_block_moe_device_routed_bf16x_f32(
            _vp(self.pool.table), N_ROUTED, self._at(self.idx, i, "idx"), self._at(self.w, i, "w"), TOP_K,
            ctypes.cast(self.pool.shared, ctypes.c_void_p), self._at(self.x, i, "x"), _vp(self.y), _vp(self.ys),
            _vp(self.ybf), _vp(self.rejected), 1, INTER, HID, math.ceil(HID / 128), math.ceil(INTER / 128))
        if code != 0:
            raise RuntimeError(f"fp8_e4m3_block_moe_device_routed_bf16x_f32 failed with code {code}")

    def fused(self, i):
        code = self.lib.fp8_e4m3_block_moe_from_logits_bf16x_f32(
            self._at(self.logits, i, "logits"), None, N_GROUPS, TOPK_GROUPS, 0, ROUTE_SCALE, _vp(self.pool.table),
            N_ROUTED, TOP_K, ctypes.cast(self.pool.shared, ctypes.c_void_p), self._at(self.x, i, "x"), _vp(self.y),
            _vp(self.ys), _vp(self.ybf), self._at(self.idx, i, "idx"), self._at(self.w, i, "w"), _vp(self.rejected),
            1, INTER, HID, math.ceil(HID / 128), math.ceil(INTER / 128))
        if code != 0:
            raise RuntimeError(f"fp8_e4m3_block_moe_from_logits_bf16x_f32 failed with code {code}")

    def step(self, i):
        self.fused(i)

    def two_calls(self, i):
        self.route(i)
        self.moe(i)


def bench_moe_layer(torch, lib, timer, steps, warmup):
    pool = MoEPool(torch)
    total = warmup + steps
    st = MoEStep(torch, lib, pool, total)
    lib.pocketlm_set_stream(_stream_ptr(torch))
    for i in range(warmup):
        st.step(i)
    torch.cuda.synchronize()
    if int(st.rejected.item()) != 0:
        raise RuntimeError("the device plan left out router indices")
    # the headline: K steps, router included
    ms_steps = timer.run([lambda i=i: st.step(warmup + i) for i in range(steps)])
    # the roofline region: the MoE layer's own launches on the same K tokens,
    # the router's outputs (already written by the timed steps) read as they are
    ms_moe = timer.run([lambda i=i: st.moe(warmup + i) for i in range(steps)])
    chosen = st.idx[warmup:].cpu()
    distinct = len(set(chosen.reshape(-1).tolist()))
    # the same steps as two calls: the router, then the device-routed MoE
    ms_two = timer.run([lambda i=i: st.two_calls(warmup + i) for i in range(steps)])
    return {"pool": pool, "step": st, "ms_per_step": ms_steps / steps, "ms_per_moe": ms_moe / steps,
            "ms_per_two_calls": ms_two / steps, "distinct_experts": distinct}


# --------------------------------------------------------------------------- verifier batch (FP8 projections)

VERIFIER_SHAPES = (("q_a", 1536, 7168), ("kv_a", 576, 7168), ("o", 7168, 16384),
                   ("expert gate/up", 2048, 7168), ("expert down", 7168, 2048))


def bench_verifier(torch, lib, timer, pool, ms=(1, 8), reps=200):
    """Each DeepSeek-V3 projection of the verifier batch at M rows of bf16
    activations, through fp8_e4m3_block_linear_bf16x_f32.  The expert shapes
    rotate over the pool's 256 experts; q_a and kv_a over the first rows of
    the pool's gate matrices (row-major, so a prefix of rows is a weight of
    its own); o over 9 copies of its own (1.06 GB), and o once more in 8-row
    tiles (fp8_e4m3_pack_tiles8 / fp8_e4m3_block_linear_tiles8_bf16x_f32, the
    same values)."""
    gen = torch.Generator(device="cuda").manual_seed(11)
    o_sets = []
    for _ in range(max(2, math.ceil(MALL_BYTES / (7168 * 16384)))):
        w = torch.randn((7168, 16384), generator=gen, device="cuda").mul_(0.02).to(torch.float8_e4m3fn)
        s = torch.rand((56, 128), generator=gen, device="cuda").mul_(9e-3).add_(1e-3)
        o_sets.append((w.view(torch.uint8), s))
    ex = pool.experts[:N_ROUTED]
    sources = {
        "q_a": [(e[0], e[1]) for e in ex],
        "kv_a": [(e[0], e[1]) for e in ex],
        "o": o_sets,
        "expert gate/up": [(e[0], e[1]) for e in ex],
        "expert down": [(e[4], e[5]) for e in ex],
    }
    out = []
    lib.pocketlm_set_stream(_stream_ptr(torch))
    tiles = []
    for w, s in o_sets:
        t = torch.empty((lib.fp8_e4m3_tiles8_bytes(7168, 16384),), dtype=torch.uint8, device="cuda")
        if lib.fp8_e4m3_pack_tiles8(_vp(w), _vp(t), 7168, 16384) != 0:
            raise RuntimeError("fp8_e4m3_pack_tiles8 failed")
        tiles.append((t, s))
    sources["o (8-row tiles)"] = tiles
    entry = {"o (8-row tiles)": "fp8_e4m3_block_linear_tiles8_bf16x_f32"}
    for name, rows, cols in VERIFIER_SHAPES + (("o (8-row tiles)", 7168, 16384),):
        sets = sources[name]
        fn_name = entry.get(name, "fp8_e4m3_block_linear_bf16x_f32")
        fn = getattr(lib, fn_name)
        for m in ms:
            x = torch.randn((m, cols), generator=gen, device="cuda").to(torch.bfloat16)
            y = torch.empty((m, rows), device="cuda")
            sc = math.ceil(cols / 128)

            def call(w, s, x=x, y=y, m=m, rows=rows, cols=cols, sc=sc, fn=fn, fn_name=fn_name):
                code = fn(_vp(w), _vp(s), _vp(x), _vp(y), m, rows, cols, sc)
                if code != 0:
                    raise RuntimeError(f"{fn_name} failed with code {code}")

            for w, s in sets[:4]:
                call(w, s)
            torch.cuda.synchronize()
            n = reps
            ms_total = timer.run([lambda j=j: call(*sets[j % len(sets)]) for j in range(n)])
            us = 1e3 * ms_total / n
            nbytes = fp8_bytes(rows, cols, m)
            gbs = nbytes / us / 1e3
            out.append({"shape": f"{name} {rows}x{cols}", "m": m, "us": round(us, 3), "bytes": nbytes,
                        "gb_s": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)})
    del o_sets, tiles, sources
    torch.cuda.empty_cache()
    return out


# --------------------------------------------------------------------------- CPU baseline

def _host_info():
    info = {"nproc": os.cpu_count()}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in txt.splitlines():
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "Model name":
                info["model"] = v
            elif k == "Socket(s)":
                info["sockets"] = int(v) if v.isdigit() else v
            elif k == "CPU(s)":
                info["cpus"] = int(v) if v.isdigit() else v
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        info["affinity"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        pass
    return info


def _ref_lib():
    """The reference's fp8_linear.cpp built from its source (oracle/_ref), or None."""
    path = REPO / "oracle" / "_ref" / "libref_fp8_linear.so"
    if not path.exists():
        return None
    lib = ctypes.CDLL(str(path))
    vp, i64 = ctypes.c_void_p, ctypes.c_longlong
    lib.fp8_e4m3_block_mlp_many_weighted_f32.argtypes = [vp] * 9 + [i64] * 6
    lib.fp8_e4m3_block_mlp_f32.argtypes = [vp] * 8 + [i64] * 5
    lib.fp8_e4m3_block_linear_f32.argtypes = [vp] * 4 + [i64] * 4
    for f in (lib.fp8_e4m3_block_mlp_many_weighted_f32, lib.fp8_e4m3_block_mlp_f32, lib.fp8_e4m3_block_linear_f32):
        f.restype = ctypes.c_int
    return lib


def _ref_row8_lib():
    """The reference's fp16_packed_gemv.cpp built from its source (oracle/_ref), or None."""
    path = REPO / "oracle" / "_ref" / "libref_fp16_packed_gemv.so"
    if not path.exists():
        return None
    lib = ctypes.CDLL(str(path))
    vp, i64 = ctypes.c_void_p, ctypes.c_longlong
    lib.native_packed_gemv_rows8.argtypes = [vp, vp, vp, i64, i64, ctypes.c_int]
    lib.native_packed_gemv_rows8.restype = ctypes.c_int
    return lib


def _omp():
    """The OpenMP runtime the reference build links (to set its thread count)."""
    gomp = ctypes.CDLL("libgomp.so.1")
    gomp.omp_set_num_threads.argtypes = [ctypes.c_int]
    gomp.omp_get_max_threads.restype = ctypes.c_int
    return gomp


def _timed_calls(fn, seconds, min_calls=2):
    n = 0
    t0 = time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= min_calls:
            return n, el


def cpu_moe_baseline(torch, r, seconds):
    """The reference's CPU MoE layer (8 routed, route-weighted + shared) on
    the experts step 0 chose, weights warm in host RAM, all threads and one."""
    import numpy as np

    st, pool = r["step"], r["pool"]
    warm = 0
    idx = st.idx[warm].cpu().tolist()
    wts = st.w[warm].cpu().tolist()
    order = sorted(range(TOP_K), key=lambda j: idx[j])  # run_fp8_moe's sorted distinct experts
    routed = [[t.cpu().numpy() for t in pool.experts[idx[j]]] for j in order]
    shared = [t.cpu().numpy() for t in pool.experts[N_ROUTED]]
    route = np.array([wts[j] for j in order], dtype=np.float32)
    hidden = st.x[warm:warm + 1].float().cpu().numpy()
    out = np.empty((1, HID), dtype=np.float32)
    out_s = np.empty((1, HID), dtype=np.float32)
    ref = _ref_lib()
    kind = "reference"
    if ref is not None:
        tabs = [np.array([e[k].ctypes.data for e in routed], dtype=np.uint64) for k in range(6)]

        def layer():
            c1 = ref.fp8_e4m3_block_mlp_many_weighted_f32(*[t.ctypes.data for t in tabs], hidden.ctypes.data,
                                                          route.ctypes.data, out.ctypes.data, TOP_K, 1, INTER,
                                                          HID, 56, 16)
            c2 = ref.fp8_e4m3_block_mlp_f32(*[t.ctypes.data for t in shared], hidden.ctypes.data, out_s.ctypes.data,
                                            1, INTER, HID, 56, 16)
            if c1 != 0 or c2 != 0:
                raise RuntimeError(f"reference MoE returned {c1}, {c2}")
    else:
        import oracle

        kind = "port"

        def layer():
            oracle.fp8_mlp_many_weighted([tuple(e) for e in routed], hidden, route)
            oracle.fp8_mlp(*shared, hidden)

    omp = _omp()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or omp.omp_get_max_threads()
    omp.omp_set_num_threads(threads)
    n_all, el_all = _timed_calls(layer, seconds)
    omp.omp_set_num_threads(1)
    n_one, el_one = _timed_calls(layer, seconds / 2)
    omp.omp_set_num_threads(threads)
    nbytes = moe_layer_bytes(1)
    us_all, us_one = el_all / n_all * 1e6, el_one / n_one * 1e6
    return {
        "value": round(nbytes / us_all / 1e3, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": kind,
        "us_per_step": round(us_all, 1),
        "sample": (f"{n_all} calls of the reference's fp8_e4m3_block_mlp_many_weighted_f32 (8 routed experts) + "
                   f"fp8_e4m3_block_mlp_f32 (shared expert), fp8_linear.cpp built from source with g++ -O2 "
                   f"-fopenmp, on the experts of the first timed token, {el_all:.1f} s on {threads} OpenMP "
                   f"threads, weights warm in host RAM" if kind == "reference" else
                   f"{n_all} calls of the oracle's restatement, {el_all:.1f} s on {threads} threads"),
        "single_thread": {"value": round(nbytes / us_one / 1e3, 3), "unit": "GB/s", "us_per_step": round(us_one, 1),
                          "calls": n_one},
        "host": _host_info(),
    }


def cpu_verifier_baseline(seconds_each=2.0):
    """The reference's fp8_e4m3_block_linear_f32 on the 7168 x 16384 output
    projection at M = 8, in both of its modes: the default (each activation
    row re-reads the weight, fp8_linear.cpp:96-116) and batch reuse (one
    pass over the weight for the whole batch, fp8_linear.cpp:68-94,
    PCKETLM_ENABLE_NATIVE_FP8_BATCH_REUSE=1)."""
    import numpy as np

    ref = _ref_lib()
    if ref is None:
        return None
    rng = np.random.default_rng(5)
    w = rng.integers(0, 0x7E, size=(7168, 16384), dtype=np.uint8)  # finite e4m3 bytes
    s = rng.uniform(1e-3, 1e-2, size=(56, 128)).astype(np.float32)
    x = rng.standard_normal((8, 16384)).astype(np.float32)
    y = np.empty((8, 7168), dtype=np.float32)
    res = {}
    old = os.environ.get("PCKETLM_ENABLE_NATIVE_FP8_BATCH_REUSE")
    try:
        for mode, flag in (("default (W re-read per row)", None), ("batch reuse (W read once)", "1")):
            if flag is None:
                os.environ.pop("PCKETLM_ENABLE_NATIVE_FP8_BATCH_REUSE", None)
            else:
                os.environ["PCKETLM_ENABLE_NATIVE_FP8_BATCH_REUSE"] = flag
            n, el = _timed_calls(lambda: ref.fp8_e4m3_block_linear_f32(w.ctypes.data, s.ctypes.data, x.ctypes.data,
                                                                        y.ctypes.data, 8, 7168, 16384, 128),
                                 seconds_each)
            us = el / n * 1e6
            res[mode] = {"us": round(us, 1), "gb_s": round(fp8_bytes(7168, 16384, 8) / us / 1e3, 3), "calls": n}
    finally:
        if old is None:
            os.environ.pop("PCKETLM_ENABLE_NATIVE_FP8_BATCH_REUSE", None)
        else:
            os.environ["PCKETLM_ENABLE_NATIVE_FP8_BATCH_REUSE"] = old
    return res


def _traffic(workload):
    """HBM bytes per step from the committed counter runs (FETCH_SIZE and
    WRITE_SIZE scaled by a plain copy's reading; profiles/traffic.json) and
    where they come from, or (None, None) when they are absent.  The counters
    are not read live: they need runs of their own under rocprofv3."""
    f = REPO / "profiles" / "traffic.json"
    if not f.exists():
        return None, None
    try:
        entry = json.loads(f.read_text()).get(workload) or {}
        src = f"profiles/traffic.json[{workload!r}]: " + (entry.get("source") or "?")
        return entry.get("bytes_per_step"), src
    except (OSError, ValueError, AttributeError):
        return None, None


def main_line(args):
    import torch

    from pocketlm_amd import _lib

    torch.cuda.set_device(0)
    lib = _lib.load()
    if lib.pocketlm_device_available() != 1:
        raise RuntimeError("libpocketlm_hip.so reports no gfx950 device")
    timer = Timer(torch)
    r = bench_moe_layer(torch, lib, timer, args.steps, args.warmup)
    ms = r["ms_per_step"]
    value = moe_step_bytes(1) / (ms / 1e3) / 1e9
    moe_ms = r["ms_per_moe"]
    achieved = moe_layer_bytes(1) / (moe_ms / 1e3) / 1e9
    traffic, traffic_src = _traffic("moe_layer")
    roof = {
        "bound": "hbm",
        "kernel": "the MoE layer's launches of fp8_e4m3_block_moe_device_routed_bf16x_f32: fp8_rows_kernel "
                  "(the plan from the router's choices, gate/up + SiLU, 8 chosen + shared expert), fp8_down_kernel "
                  "(down, route-weighted sum, shared expert, bf16 output)",
        "achieved": round(achieved, 2),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBS, 4),
        "traffic": traffic,
        "traffic_unit": "HBM bytes per MoE layer call (all its launches)",
        "traffic_source": traffic_src,
        "us_per_launch_group": round(1e3 * moe_ms, 3),
        "bytes_per_launch_group": moe_layer_bytes(1),
    }
    ver = bench_verifier(torch, lib, timer, r["pool"])
    o8 = next(v for v in ver if v["shape"].startswith("o ") and v["m"] == 8)
    m8 = {"workload": "speculative / MTP verifier batch: FP8 output projection 7168x16384, M=8 bf16 rows, "
                      "fp8_e4m3_block_linear_bf16x_f32 (each weight byte read once per batch)",
          "us": o8["us"], "value": o8["gb_s"], "unit": "GB/s", "frac": o8["frac"], "bytes": o8["bytes"]}
    cpu = None
    if not args.no_cpu:
        cpu = cpu_moe_baseline(torch, r, args.cpu_seconds)
        cv = cpu_verifier_baseline()
        if cv is not None:
            m8["cpu_reference"] = {"kind": "reference", "threads": cpu["cores"], **{k: v for k, v in cv.items()}}
    line = {
        "metric": "dequant-GEMV µs & achieved HBM GB/s (% of peak) at M=1 and M=8",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_step": round(1e3 * ms, 3),
        "us_per_step_router_then_moe": round(1e3 * r["ms_per_two_calls"], 3),
        "pct_of_peak": round(100 * value / PEAK_HBM_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8 e4m3 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic (e4m3 weights from N(0,0.02), scale_inv ~U(1e-3,1e-2), router logits and hidden ~N(0,1))",
        "config": {
            "workload": "DeepSeek-V3 MoE layer decode, M=1: hidden 7168, 256 routed + 1 shared expert resident "
                        "(11.3 GB), moe_inter 2048, sigmoid routing (8 groups keep 4, top 8, x2.5) on fresh logits "
                        "per token, SwiGLU, bf16 output; step = fp8_e4m3_block_moe_from_logits_bf16x_f32 "
                        "(route + plan, gate/up, down)",
            "bytes_per_step": moe_step_bytes(1),
            "distinct_experts_in_timed_steps": r["distinct_experts"],
        },
        "roofline": roof,
        "cpu_baseline": cpu,
        "m8": m8,
        "verifier": ver,
    }
    print(json.dumps(line), flush=True)


# --------------------------------------------------------------------------- Q4 workloads (table)

def _q4_sets(torch, fmt, shapes, nsets, seed=20261201):
    """nsets copies of Q4 matrices of the given [rows, cols] shapes (device)."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    sets = []
    for _ in range(nsets):
        mats = []
        for rows, cols in shapes:
            w = torch.randn((rows, cols), generator=gen, device="cuda", dtype=torch.float32).mul_(0.02).to(torch.float16)
            packed, scales, _ = fmt.quantize_tensor_to_q4(w)
            del w
            mats.append((packed, scales, rows, cols))
        sets.append(mats)
    torch.cuda.synchronize()
    return sets


def q4_bytes(rows, cols):
    # packed weights + fp16 scales + fp16 x + fp32 y
    return rows * cols // 2 + 2 * rows + 2 * cols + 4 * rows


def mlp_bytes(hidden, inter):
    """Algorithmic HBM bytes of one Q4 SwiGLU MLP call: the three packed
    matrices and their fp16 row scales, the fp16 input and output, and the
    intermediate written once by the gate/up kernel and read once by the down
    kernel (4 bytes per value each way).  The implementation also keeps an
    fp32 copy of the intermediate for its exact fallback; those bytes show up
    in the measured traffic, not here."""
    weights = 3 * hidden * inter // 2
    scales = 2 * (2 * inter + hidden)
    return weights + scales + 2 * hidden + 2 * hidden + 2 * 4 * inter


def bench_q4_mlp(torch, lib, fmt, steps, warmup, timer, hidden=3584, inter=18944):
    """One step = one call of the reference's Q4 MLP entry point
    (q4_moe_selected_forward_u16 with one selected expert, route weight 1.0):
    gate/up [inter, hidden] + SiLU, then down [hidden, inter]."""
    shapes = [(inter, hidden), (inter, hidden), (hidden, inter)]
    per_set = sum(r * c // 2 for r, c in shapes)
    nsets = max(2, math.ceil(MALL_BYTES / per_set))
    sets = _q4_sets(torch, fmt, shapes, nsets)
    gen = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn((hidden,), generator=gen, device="cuda").to(torch.float16)
    route = torch.ones(1, device="cuda")
    out = torch.empty((hidden,), device="cuda", dtype=torch.float16)
    lib.pocketlm_set_stream(_stream_ptr(torch))
    calls = []
    for mats in sets:
        tables = [(ctypes.c_void_p * 1)(t.data_ptr()) for m in mats for t in m[:2]]
        calls.append(tuple(ctypes.cast(t, ctypes.c_void_p) for t in tables))

    def launch(tabs):
        code = lib.q4_moe_selected_forward_u16(ctypes.c_void_p(x.data_ptr()), *tabs,
                                               ctypes.c_void_p(route.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                               hidden, inter, 1)
        if code != 0:
            raise RuntimeError(f"q4_moe_selected_forward_u16 failed with code {code}")

    for i in range(warmup):
        launch(calls[i % nsets])
    torch.cuda.synchronize()
    launches = [lambda t=calls[i % nsets]: launch(t) for i in range(steps)]
    t0 = time.perf_counter()
    total_ms = timer.run(launches, hold_ms=max(30.0, 0.05 * len(launches)))
    wall = time.perf_counter() - t0
    return {
        "total_ms": total_ms,
        "ms_per_step": total_ms / steps,
        "step_bytes": mlp_bytes(hidden, inter),
        "wall_s": wall,
        "nsets": nsets,
        "host_set": sets[0],
        "x": x,
        "hidden": hidden,
        "inter": inter,
    }


# --------------------------------------------------------------------------- table mode

def table(args):
    import numpy as np
    import torch

    from pocketlm_amd import _lib, formats, native

    torch.cuda.set_device(0)
    lib = _lib.load()
    timer = Timer(torch)
    rows_out = []
    only = [t for t in (args.only or "").split(",") if t]

    def want(*names):
        return not only or any(t in n for n in names for t in only)

    ref8, refr8 = _ref_lib(), _ref_row8_lib()
    omp = _omp()
    all_threads = omp.omp_get_max_threads()
    os.environ.pop("PCKETLM_NATIVE_THREADS", None)
    os.environ.pop("PCKETLM_ENABLE_NATIVE_FP8_BATCH_REUSE", None)  # the reference's default mode

    def cpu_time(fn):
        t0 = time.perf_counter()
        n = 0
        while True:
            fn()
            n += 1
            if time.perf_counter() - t0 > 1.5:
                break
        return (time.perf_counter() - t0) / n * 1e6

    def measure(name, m, make_calls, nbytes, cpu_fn=None, cpu_kind="port", ref_fn=None):
        """ref_fn: the reference's own compiled code (oracle/_ref) for this
        row, timed with all threads and with one; cpu_fn (the oracle's
        restatement) only where the reference build has no such entry."""
        if not want(name):
            return
        calls = make_calls()
        for fn in calls[: min(len(calls), 8)]:
            code = fn()
            if isinstance(code, int) and code != 0:
                raise RuntimeError(f"{name}: entry point failed with code {code} ({_lib.last_error()})")
        torch.cuda.synchronize()
        reps = max(20, min(400, int(5e9 // max(nbytes, 1))))
        launches = [calls[i % len(calls)] for i in range(reps)]
        med = timer.run(launches, hold_ms=max(30.0, 0.05 * len(launches))) / reps
        gbs = nbytes / (med / 1e3) / 1e9
        cpu_us = cpu_gbs = cpu1_us = None
        if ref_fn is not None and not args.no_cpu:
            cpu_kind = "reference"
            omp.omp_set_num_threads(all_threads)
            cpu_us = cpu_time(ref_fn)
            omp.omp_set_num_threads(1)
            cpu1_us = cpu_time(ref_fn)
            omp.omp_set_num_threads(all_threads)
            cpu_gbs = nbytes / (cpu_us / 1e6) / 1e9
        elif cpu_fn is not None and not args.no_cpu:
            cpu_us = cpu_time(cpu_fn)
            cpu_gbs = nbytes / (cpu_us / 1e6) / 1e9
        rows_out.append((name, m, 1e3 * med, gbs, 100 * gbs / PEAK_HBM_GBS, cpu_us, cpu_gbs, cpu_kind, cpu1_us))
        print(f"{name:40s} M={m}  {1e3 * med:9.2f} us  {gbs:8.1f} GB/s  {100 * gbs / PEAK_HBM_GBS:5.1f}%"
              + (f"   cpu {cpu_us:10.1f} us {cpu_gbs:7.2f} GB/s {cpu_kind}" if cpu_us else "")
              + (f" (1 thread {cpu1_us:10.1f} us)" if cpu1_us else ""), flush=True)

    import oracle
    from oracle import mla as oracle_mla

    gen = torch.Generator(device="cuda").manual_seed(11)

    def fp8_sets(rows, cols, count):
        out = []
        for _ in range(count):
            w = torch.randn((rows, cols), generator=gen, device="cuda").mul_(0.02).to(torch.float8_e4m3fn)
            w = w.view(torch.uint8)
            s = torch.rand((math.ceil(rows / 128), math.ceil(cols / 128)), generator=gen, device="cuda") * 9e-3 + 1e-3
            out.append((w, s))
        return out

    # ---- FP8 linear shapes (configs 1 and 5)
    for name, rows, cols in (("fp8 linear 2048x7168", 2048, 7168), ("fp8 q_a 1536x7168", 1536, 7168),
                             ("fp8 kv_a 576x7168", 576, 7168), ("fp8 o 7168x16384", 7168, 16384),
                             ("fp8 expert gate/up 2048x7168", 2048, 7168), ("fp8 expert down 7168x2048", 7168, 2048)):
        if not want(name):
            continue
        count = max(2, math.ceil(MALL_BYTES / (rows * cols)))
        sets = fp8_sets(rows, cols, count)
        host_w, host_s = sets[0][0].cpu().numpy(), sets[0][1].cpu().numpy()
        for m in (1, 2, 4, 8):
            if name.startswith("fp8 linear") and m > 1:
                continue
            # bf16 activations, as the configuration states, through the bf16 twin
            # of the linear (the same values as widening them to fp32 first)
            x = torch.randn((m, cols), generator=gen, device="cuda").to(torch.bfloat16)
            y = torch.empty((m, rows), device="cuda")
            lib.pocketlm_set_stream(_stream_ptr(torch))

            def make(sets=sets, x=x, y=y, rows=rows, cols=cols, m=m):
                return [lambda w=w, s=s: lib.fp8_e4m3_block_linear_bf16x_f32(
                    ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(s.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                    ctypes.c_void_p(y.data_ptr()), m, rows, cols, math.ceil(cols / 128)) for w, s in sets]

            xh = x.float().cpu().numpy()
            yh = np.empty((m, rows), dtype=np.float32)
            measure(name, m, make, fp8_bytes(rows, cols, m),
                    lambda w=host_w, s=host_s, xh=xh: oracle.fp8_linear(w, s, xh, batch_reuse=True),
                    ref_fn=None if ref8 is None else
                    lambda w=host_w, s=host_s, xh=xh, yh=yh, m=m, rows=rows, cols=cols: ref8.fp8_e4m3_block_linear_f32(
                        w.ctypes.data, s.ctypes.data, xh.ctypes.data, yh.ctypes.data, m, rows, cols, s.shape[1]))
        del sets
        torch.cuda.empty_cache()

    # ---- the o projection through the reference-ABI entry point, whose
    # activations are fp32 (bf16 values widened, as the reference's wrapper
    # passes them: src/pcketlm/native/__init__.py:3442-3476)
    if want("fp8 o 7168x16384 (fp32 activations)"):
        rows, cols = 7168, 16384
        count = max(2, math.ceil(MALL_BYTES / (rows * cols)))
        sets = fp8_sets(rows, cols, count)
        host_w, host_s = sets[0][0].cpu().numpy(), sets[0][1].cpu().numpy()
        for m in (1, 8):
            x = torch.randn((m, cols), generator=gen, device="cuda").to(torch.bfloat16).float()
            y = torch.empty((m, rows), device="cuda")
            lib.pocketlm_set_stream(_stream_ptr(torch))

            def make(sets=sets, x=x, y=y, m=m):
                return [lambda w=w, s=s: lib.fp8_e4m3_block_linear_f32(
                    ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(s.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                    ctypes.c_void_p(y.data_ptr()), m, rows, cols, cols // 128) for w, s in sets]

            xh = x.cpu().numpy()
            yh = np.empty((m, rows), dtype=np.float32)
            measure("fp8 o 7168x16384 (fp32 activations)", m, make, fp8_bytes(rows, cols, m) + 2 * m * cols,
                    lambda w=host_w, s=host_s, xh=xh: oracle.fp8_linear(w, s, xh, batch_reuse=True),
                    ref_fn=None if ref8 is None else
                    lambda w=host_w, s=host_s, xh=xh, yh=yh, m=m: ref8.fp8_e4m3_block_linear_f32(
                        w.ctypes.data, s.ctypes.data, xh.ctypes.data, yh.ctypes.data, m, rows, cols, s.shape[1]))
        del sets
        torch.cuda.empty_cache()

    # ---- the o projection with its weight in 8-row tiles (packed once; the
    # same values as the row-major linear)
    if want("fp8 o 7168x16384 (8-row tiles)"):
        rows, cols = 7168, 16384
        count = max(2, math.ceil(MALL_BYTES / (rows * cols)))
        sets = fp8_sets(rows, cols, count)
        host_w, host_s = sets[0][0].cpu().numpy(), sets[0][1].cpu().numpy()
        packed = []
        for w, s in sets:
            t = torch.empty((lib.fp8_e4m3_tiles8_bytes(rows, cols),), dtype=torch.uint8, device="cuda")
            if lib.fp8_e4m3_pack_tiles8(ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(t.data_ptr()), rows, cols):
                raise RuntimeError("fp8_e4m3_pack_tiles8 failed")
            packed.append((t, s))
        del sets
        for m in (1, 2, 4, 8):
            x = torch.randn((m, cols), generator=gen, device="cuda").to(torch.bfloat16)
            y = torch.empty((m, rows), device="cuda")
            lib.pocketlm_set_stream(_stream_ptr(torch))

            def make(x=x, y=y, m=m):
                return [lambda t=t, s=s: lib.fp8_e4m3_block_linear_tiles8_bf16x_f32(
                    ctypes.c_void_p(t.data_ptr()), ctypes.c_void_p(s.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                    ctypes.c_void_p(y.data_ptr()), m, rows, cols, cols // 128) for t, s in packed]

            xh = x.float().cpu().numpy()
            yh = np.empty((m, rows), dtype=np.float32)
            measure("fp8 o 7168x16384 (8-row tiles)", m, make, fp8_bytes(rows, cols, m),
                    lambda w=host_w, s=host_s, xh=xh: oracle.fp8_linear(w, s, xh, batch_reuse=True),
                    ref_fn=None if ref8 is None else
                    lambda w=host_w, s=host_s, xh=xh, yh=yh, m=m: ref8.fp8_e4m3_block_linear_f32(
                        w.ctypes.data, s.ctypes.data, xh.ctypes.data, yh.ctypes.data, m, rows, cols, s.shape[1]))
        del packed
        torch.cuda.empty_cache()

    # ---- q_a and kv_a from one hidden state in one launch (configuration 5's
    # attention input projections)
    if want("fp8 q_a + kv_a"):
        count = max(2, math.ceil(MALL_BYTES / ((1536 + 576) * 7168)))
        qa, kva = fp8_sets(1536, 7168, count), fp8_sets(576, 7168, count)
        hq = (qa[0][0].cpu().numpy(), qa[0][1].cpu().numpy(), kva[0][0].cpu().numpy(), kva[0][1].cpu().numpy())
        rows_arr = (ctypes.c_int64 * 2)(1536, 576)
        for m in (1, 2, 4, 8):
            x = torch.randn((m, 7168), generator=gen, device="cuda").to(torch.bfloat16)
            yq, yk = torch.empty((m, 1536), device="cuda"), torch.empty((m, 576), device="cuda")
            outs_arr = (ctypes.c_uint64 * 2)(yq.data_ptr(), yk.data_ptr())
            tabs = [((ctypes.c_uint64 * 2)(a[0].data_ptr(), b[0].data_ptr()),
                     (ctypes.c_uint64 * 2)(a[1].data_ptr(), b[1].data_ptr())) for a, b in zip(qa, kva)]
            lib.pocketlm_set_stream(_stream_ptr(torch))

            def make(tabs=tabs, x=x, outs_arr=outs_arr, m=m):
                return [lambda t=t: lib.fp8_e4m3_block_linear_many_bf16x_f32(
                    ctypes.cast(t[0], ctypes.c_void_p), ctypes.cast(t[1], ctypes.c_void_p), ctypes.c_void_p(x.data_ptr()),
                    ctypes.cast(outs_arr, ctypes.c_void_p), ctypes.cast(rows_arr, ctypes.c_void_p), 2, m, 7168, 56)
                    for t in tabs]

            xh = x.float().cpu().numpy()
            yq_h, yk_h = np.empty((m, 1536), dtype=np.float32), np.empty((m, 576), dtype=np.float32)
            measure("fp8 q_a + kv_a (one launch)", m, make,
                    fp8_bytes(1536, 7168, m) + fp8_bytes(576, 7168, m) - 2 * m * 7168,
                    lambda xh=xh: (oracle.fp8_linear(hq[0], hq[1], xh, batch_reuse=True),
                                   oracle.fp8_linear(hq[2], hq[3], xh, batch_reuse=True)),
                    ref_fn=None if ref8 is None else
                    lambda xh=xh, m=m: (
                        ref8.fp8_e4m3_block_linear_f32(hq[0].ctypes.data, hq[1].ctypes.data, xh.ctypes.data,
                                                       yq_h.ctypes.data, m, 1536, 7168, 56),
                        ref8.fp8_e4m3_block_linear_f32(hq[2].ctypes.data, hq[3].ctypes.data, xh.ctypes.data,
                                                       yk_h.ctypes.data, m, 576, 7168, 56)))
        del qa, kva
        torch.cuda.empty_cache()

    # ---- FP8 dequant (config 1 matrix)
    sets = fp8_sets(2048, 7168, 24) if want("fp8 dequant") else []
    out16 = torch.empty((2048, 7168), device="cuda", dtype=torch.float16)
    lib.pocketlm_set_stream(_stream_ptr(torch))
    hw, hs = (sets[0][0].cpu().numpy(), sets[0][1].cpu().numpy()) if sets else (None, None)
    measure("fp8 dequant->fp16 2048x7168", 1,
            lambda: [lambda w=w, s=s: lib.fp8_e4m3_dequant_to_fp16(ctypes.c_void_p(w.data_ptr()),
                                                                 ctypes.c_void_p(s.data_ptr()),
                                                                 ctypes.c_void_p(out16.data_ptr()), 2048, 7168, 56)
                     for w, s in sets],
            2048 * 7168 * 3 + 4 * 16 * 56, lambda: oracle.fp8_dequant(hw, hs, "f16"))
    del sets
    torch.cuda.empty_cache()

    # ---- Q4 (config 2)
    shapes = [(18944, 3584), (18944, 3584), (3584, 18944)]
    qsets = _q4_sets(torch, formats, shapes, 10 if want("q4") else 1)
    xq = torch.randn((3584,), generator=gen, device="cuda").to(torch.float16)
    xd = torch.randn((18944,), generator=gen, device="cuda").to(torch.float16)
    yq = torch.empty((18944,), device="cuda")
    lib.pocketlm_set_stream(_stream_ptr(torch))
    for j, label in ((0, "q4 gemv gate/up 18944x3584"), (2, "q4 gemv down 3584x18944")):
        rows, cols = shapes[j]
        xx = xq if cols == 3584 else xd
        hp = qsets[0][j][0].cpu().numpy()
        hsc = qsets[0][j][1].cpu().view(torch.int16).numpy().view(np.uint16)
        hx = xx.float().cpu().numpy()
        measure(label, 1, lambda j=j, rows=rows, cols=cols, xx=xx: [
            lambda p=s[j][0], sc=s[j][1]: lib.q4_gemv_f16_f32(ctypes.c_void_p(p.data_ptr()),
                                                             ctypes.c_void_p(sc.data_ptr()),
                                                             ctypes.c_void_p(xx.data_ptr()),
                                                             ctypes.c_void_p(yq.data_ptr()), rows, cols)
            for s in qsets], q4_bytes(rows, cols),
            lambda hp=hp, hsc=hsc, hx=hx, rows=rows, cols=cols: oracle.q4_gemv(hp, hsc, hx, rows, cols))
    # Q4 SwiGLU MLP through the reference entry point (one expert, route 1.0)
    route = torch.ones(1, device="cuda")
    outh = torch.empty((3584,), device="cuda", dtype=torch.float16)
    arrs = []
    for s in qsets:
        a = [(ctypes.c_void_p * 1)(s[0][0].data_ptr()), (ctypes.c_void_p * 1)(s[0][1].data_ptr()),
             (ctypes.c_void_p * 1)(s[1][0].data_ptr()), (ctypes.c_void_p * 1)(s[1][1].data_ptr()),
             (ctypes.c_void_p * 1)(s[2][0].data_ptr()), (ctypes.c_void_p * 1)(s[2][1].data_ptr())]
        arrs.append(a)
    mlp_bytes = sum(r * c // 2 + 2 * r for r, c in shapes) + 2 * 3584 + 2 * 3584
    hexp = [(qsets[0][0][0].cpu().numpy(), qsets[0][0][1].cpu().view(torch.int16).numpy().view(np.uint16),
             qsets[0][1][0].cpu().numpy(), qsets[0][1][1].cpu().view(torch.int16).numpy().view(np.uint16),
             qsets[0][2][0].cpu().numpy(), qsets[0][2][1].cpu().view(torch.int16).numpy().view(np.uint16))]
    hx16 = xq.cpu().view(torch.int16).numpy().view(np.uint16)
    measure("q4 SwiGLU MLP (2 kernels)", 1, lambda: [
        lambda a=a: lib.q4_moe_selected_forward_u16(ctypes.c_void_p(xq.data_ptr()),
                                                    *[ctypes.cast(t, ctypes.c_void_p) for t in a],
                                                    ctypes.c_void_p(route.data_ptr()),
                                                    ctypes.c_void_p(outh.data_ptr()), 3584, 18944, 1)
        for a in arrs], mlp_bytes,
        lambda: oracle.q4_moe_selected(hx16, hexp, np.ones(1, np.float32), 3584, 18944))
    outd = torch.empty((18944 * 3584,), device="cuda", dtype=torch.float16)
    measure("q4 dequant->fp16 18944x3584", 1, lambda: [
        lambda p=s[0][0], sc=s[0][1]: lib.q4_dequant_to_fp16(ctypes.c_void_p(p.data_ptr()),
                                                            ctypes.c_void_p(sc.data_ptr()),
                                                            ctypes.c_void_p(outd.data_ptr()), 18944, 3584)
        for s in qsets], 18944 * 3584 // 2 + 2 * 18944 + 2 * 18944 * 3584,
        lambda: oracle.q4_dequant_f16(hexp[0][0], hexp[0][1], 18944, 3584))
    del qsets, outd
    torch.cuda.empty_cache()

    # ---- row8 (config 3)
    for name, rows, cols in (("row8 q/o 3584x3584", 3584, 3584), ("row8 k/v 512x3584", 512, 3584),
                             ("row8 gate/up 18944x3584", 18944, 3584), ("row8 down 3584x18944", 3584, 18944)):
        if not want(name, name.replace("row8", "row8 f32-x")):
            continue
        count = max(2, math.ceil(MALL_BYTES / (2 * rows * cols)))
        packs = []
        for _ in range(count):
            w = torch.randn((rows, cols), generator=gen, device="cuda").mul_(0.02).to(torch.float16)
            packs.append(native.pack_weight_rows8(w))
            del w
        h = torch.randn((cols,), generator=gen, device="cuda").to(torch.float16)
        y = torch.empty((rows,), device="cuda")
        lib.pocketlm_set_stream(_stream_ptr(torch))
        hp = packs[0].cpu().view(torch.int16).numpy().view(np.uint16)
        hh = h.cpu().view(torch.int16).numpy().view(np.uint16)
        yh = np.empty((rows,), dtype=np.float32)
        # the reference's packed GEMV takes u16 activations: its wrapper casts fp32 ones to fp16
        ref_row8 = None if refr8 is None else (
            lambda hp=hp, hh=hh, yh=yh, rows=rows, cols=cols: refr8.native_packed_gemv_rows8(
                hh.ctypes.data, hp.ctypes.data, yh.ctypes.data, rows, cols, 0))
        measure(name, 1, lambda packs=packs, h=h, y=y, rows=rows, cols=cols: [
            lambda p=p: lib.native_packed_gemv_rows8(ctypes.c_void_p(h.data_ptr()), ctypes.c_void_p(p.data_ptr()),
                                                     ctypes.c_void_p(y.data_ptr()), rows, cols, 0) for p in packs],
            2 * math.ceil(rows / 8) * 8 * cols + 2 * cols + 4 * rows,
            lambda hp=hp, hh=hh, rows=rows, cols=cols: oracle.packed_gemv_rows8(hh, hp, rows, cols, 0),
            ref_fn=ref_row8)
        if rows == 3584:  # o-proj and down-proj also run on fp32 activations
            hf = h.float()
            hhf = hf.cpu().numpy()
            measure(name.replace("row8", "row8 f32-x"), 1, lambda packs=packs, hf=hf, y=y, rows=rows, cols=cols: [
                lambda p=p: lib.native_packed_gemv_rows8_f32_hidden(ctypes.c_void_p(hf.data_ptr()),
                                                                    ctypes.c_void_p(p.data_ptr()),
                                                                    ctypes.c_void_p(y.data_ptr()), rows, cols, 0)
                for p in packs],
                2 * math.ceil(rows / 8) * 8 * cols + 4 * cols + 4 * rows,
                lambda hp=hp, hhf=hhf, rows=rows, cols=cols: oracle.packed_gemv_rows8_f32_hidden(hhf, hp, rows, cols, 0),
                ref_fn=None if refr8 is None else
                lambda hp=hp, hhf=hhf, yh=yh, rows=rows, cols=cols: refr8.native_packed_gemv_rows8(
                    hhf.astype(np.float16).view(np.uint16).ctypes.data, hp.ctypes.data, yh.ctypes.data, rows, cols, 0))
        del packs
        torch.cuda.empty_cache()

    def dense_layer():
        # ---- row8 dense decode layer (config 3) as the decode calls it: q/k/v in one
        # launch, o on the fp32 attention output, gate/up in one launch, down on the
        # fp32 intermediate (Qwen2.5-7B: 466 MB of packed weights per layer)
        H, I, KV = 3584, 18944, 512
        shapes = {"q": (H, H), "k": (KV, H), "v": (KV, H), "o": (H, H), "gate": (I, H), "up": (I, H), "down": (H, I)}

        def packed(rows, cols):
            w = torch.randn((rows, cols), generator=gen, device="cuda").mul_(0.02).to(torch.float16)
            p = native.pack_weight_rows8(w)
            del w
            return p

        dense = [{k: packed(*v) for k, v in shapes.items()} for _ in range(3)]  # 3 x 466 MB
        h16 = torch.randn((H,), generator=gen, device="cuda").to(torch.float16)
        attn = torch.randn((H,), generator=gen, device="cuda")
        act = torch.randn((I,), generator=gen, device="cuda")
        outs = {k: torch.empty((v[0],), device="cuda") for k, v in shapes.items()}
        lib.pocketlm_set_stream(_stream_ptr(torch))

        def many(layer, names):
            pp = (ctypes.c_void_p * len(names))(*[layer[n].data_ptr() for n in names])
            bp = (ctypes.c_void_p * len(names))()
            op = (ctypes.c_void_p * len(names))(*[outs[n].data_ptr() for n in names])
            rr = (ctypes.c_longlong * len(names))(*[shapes[n][0] for n in names])
            keep = (pp, bp, op, rr)
            return lambda keep=keep: lib.native_packed_gemv_rows8_many(
                ctypes.c_void_p(h16.data_ptr()), ctypes.cast(keep[0], ctypes.c_void_p), ctypes.cast(keep[1], ctypes.c_void_p),
                ctypes.cast(keep[2], ctypes.c_void_p), ctypes.cast(keep[3], ctypes.c_void_p), len(names), H, 0)

        def f32x(layer, name, x):
            rows, cols = shapes[name]
            return lambda: lib.native_packed_gemv_rows8_f32_hidden(ctypes.c_void_p(x.data_ptr()),
                                                                   ctypes.c_void_p(layer[name].data_ptr()),
                                                                   ctypes.c_void_p(outs[name].data_ptr()), rows, cols, 0)

        def wbytes(names):
            return sum(2 * math.ceil(shapes[n][0] / 8) * 8 * shapes[n][1] + 4 * shapes[n][0] for n in names)

        host = {k: dense[0][k].cpu().view(torch.int16).numpy().view(np.uint16) for k in shapes}
        hh16 = h16.cpu().view(torch.int16).numpy().view(np.uint16)
        hattn, hact = attn.cpu().numpy(), act.cpu().numpy()

        def cpu_many(names):
            return lambda: [oracle.packed_gemv_rows8(hh16, host[n], shapes[n][0], shapes[n][1], 0) for n in names]

        hout = {k: np.empty((v[0],), dtype=np.float32) for k, v in shapes.items()}
        hattn16, hact16 = hattn.astype(np.float16).view(np.uint16), hact.astype(np.float16).view(np.uint16)

        def ref_gemv(name, x16):
            rows, cols = shapes[name]
            return refr8.native_packed_gemv_rows8(x16.ctypes.data, host[name].ctypes.data, hout[name].ctypes.data,
                                                  rows, cols, 0)

        def ref_many(names):
            return None if refr8 is None else (lambda: [ref_gemv(n, hh16) for n in names])

        measure("row8 q/k/v (one launch)", 1, lambda: [many(l, ["q", "k", "v"]) for l in dense],
                wbytes(["q", "k", "v"]) + 2 * H, cpu_many(["q", "k", "v"]), ref_fn=ref_many(["q", "k", "v"]))
        measure("row8 gate/up (one launch)", 1, lambda: [many(l, ["gate", "up"]) for l in dense],
                wbytes(["gate", "up"]) + 2 * H, cpu_many(["gate", "up"]), ref_fn=ref_many(["gate", "up"]))

        def layer_calls():
            out = []
            for l in dense:
                out += [many(l, ["q", "k", "v"]), f32x(l, "o", attn), many(l, ["gate", "up"]), f32x(l, "down", act)]
            return out

        def cpu_layer():
            cpu_many(["q", "k", "v"])()
            oracle.packed_gemv_rows8_f32_hidden(hattn, host["o"], H, H, 0)
            cpu_many(["gate", "up"])()
            oracle.packed_gemv_rows8_f32_hidden(hact, host["down"], H, I, 0)

        layer_bytes = wbytes(list(shapes)) + 2 * H * 2 + 4 * H + 4 * I
        calls = layer_calls()
        for fn in calls:
            fn()
        torch.cuda.synchronize()
        launches = [calls[i % len(calls)] for i in range(4 * 30)]
        med = timer.run(launches) / 30
        gbs = layer_bytes / (med / 1e3) / 1e9
        def ref_layer():
            for n in ("q", "k", "v"):
                ref_gemv(n, hh16)
            ref_gemv("o", hattn16)
            for n in ("gate", "up"):
                ref_gemv(n, hh16)
            ref_gemv("down", hact16)

        cpu_us = cpu_gbs = cpu1_us = None
        kind = "port"
        if not args.no_cpu:
            if refr8 is not None:
                kind = "reference"
                cpu_us = cpu_time(ref_layer)
                omp.omp_set_num_threads(1)
                cpu1_us = cpu_time(ref_layer)
                omp.omp_set_num_threads(all_threads)
            else:
                cpu_us = cpu_time(cpu_layer)
            cpu_gbs = layer_bytes / (cpu_us / 1e6) / 1e9
        print(f"{'row8 dense layer (4 launches)':40s} M=1  {1e3 * med:9.2f} us  {gbs:8.1f} GB/s  "
              f"{100 * gbs / PEAK_HBM_GBS:5.1f}%", flush=True)
        rows_out.append(("row8 dense layer (4 launches)", 1, 1e3 * med, gbs, 100 * gbs / PEAK_HBM_GBS, cpu_us, cpu_gbs,
                         kind, cpu1_us))
        del dense, host
        torch.cuda.empty_cache()

    if want("row8 dense", "row8 q/k/v (one", "row8 gate/up (one"):
        dense_layer()

    def moe_layer():
        # ---- DeepSeek-V3 MoE layer decode (config 4): 8 routed (weighted) + shared MLP
        def expert():
            g = fp8_sets(2048, 7168, 1)[0]
            u = fp8_sets(2048, 7168, 1)[0]
            d = fp8_sets(7168, 2048, 1)[0]
            return (g[0], g[1], u[0], u[1], d[0], d[1])

        layers = [[expert() for _ in range(9)] for _ in range(3)]  # 3 x 396 MB
        x = torch.randn((1, 7168), generator=gen, device="cuda").to(torch.bfloat16)  # bf16 hidden state
        logits = torch.randn((1, 256), generator=gen, device="cuda")
        _idx, rw = native.route_deepseek(logits)
        rw = rw.float().reshape(-1).contiguous()
        y = torch.empty((1, 7168), device="cuda")
        ys = torch.empty((1, 7168), device="cuda")
        lib.pocketlm_set_stream(_stream_ptr(torch))
        # one call per layer: the 8 routed experts (route-weighted sum) and the
        # shared expert (its own output) in one gate/up and one down launch
        moe_tables = [[(ctypes.c_uint64 * 9)(*[t[i].data_ptr() for t in layer]) for i in range(6)] for layer in layers]
        calls = [lambda t=tables: lib.fp8_e4m3_block_mlp_many_weighted_shared_bf16x_f32(
            *[ctypes.cast(a, ctypes.c_void_p) for a in t], ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(rw.data_ptr()),
            ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(ys.data_ptr()), 8, 1, 2048, 7168, 56, 16)
            for tables in moe_tables]

        per_expert = 3 * 2048 * 7168 + 3 * 4 * 16 * 56
        for fn in calls:
            if fn() != 0:
                raise RuntimeError("fp8_e4m3_block_mlp_many_weighted_shared_bf16x_f32 failed")
        torch.cuda.synchronize()
        launches = [calls[i % len(calls)] for i in range(30)]
        med = timer.run(launches) / len(launches)
        nbytes = 9 * per_expert + 2 * 7168 * 4
        gbs = nbytes / (med / 1e3) / 1e9
        print(f"{'ds-v3 MoE layer (8 routed + shared, 2 launches)':40s} M=1  {1e3 * med:9.2f} us  {gbs:8.1f} GB/s  "
              f"{100 * gbs / PEAK_HBM_GBS:5.1f}%", flush=True)
        # the same layers with the experts chosen on the device: a table of all
        # 256 expert slots per layer (the router's 8 filled), the router's
        # device outputs, a plan launch, the two MoE launches and the bf16 tail
        idx_dev = _idx.reshape(1, -1).contiguous()
        dev_tables = []
        for layer in layers:
            addr = torch.zeros((6, 256), dtype=torch.int64)
            for j, e in enumerate(idx_dev[0].tolist()):
                for r in range(6):
                    addr[r, e] = layer[j][r].data_ptr()
            dev_tables.append((addr.cuda(), (ctypes.c_uint64 * 6)(*[t.data_ptr() for t in layer[8]])))
        ybf = torch.empty((1, 7168), dtype=torch.bfloat16, device="cuda")
        rejected = torch.zeros((1,), dtype=torch.int32, device="cuda")
        dev_calls = [lambda t=t: lib.fp8_e4m3_block_moe_device_routed_bf16x_f32(
            ctypes.c_void_p(t[0].data_ptr()), 256, ctypes.c_void_p(idx_dev.data_ptr()), ctypes.c_void_p(rw.data_ptr()),
            8, ctypes.cast(t[1], ctypes.c_void_p), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()),
            ctypes.c_void_p(ys.data_ptr()), ctypes.c_void_p(ybf.data_ptr()), ctypes.c_void_p(rejected.data_ptr()),
            1, 2048, 7168, 56, 16) for t in dev_tables]
        for fn in dev_calls:
            if fn() != 0:
                raise RuntimeError("fp8_e4m3_block_moe_device_routed_bf16x_f32 failed")
        torch.cuda.synchronize()
        if int(rejected.item()) != 0:
            raise RuntimeError("the device plan left out router indices")
        dev_launches = [dev_calls[i % len(dev_calls)] for i in range(30)]
        dev_med = timer.run(dev_launches) / len(dev_launches)
        dev_gbs = nbytes / (dev_med / 1e3) / 1e9
        dev_name = "ds-v3 MoE layer, device-routed (2 launches, bf16 output)"
        print(f"{dev_name:40s} M=1  {1e3 * dev_med:9.2f} us  {dev_gbs:8.1f} GB/s  {100 * dev_gbs / PEAK_HBM_GBS:5.1f}%",
              flush=True)
        cpu_us = cpu_gbs = cpu1_us = None
        moe_kind = "port"
        if not args.no_cpu:
            # the weighted many-expert MLP plus the shared expert's MLP on one layer:
            # the reference's build (fp8_linear.cpp:212, 475), else the oracle's restatement
            routed = [tuple(t.cpu().numpy() for t in e) for e in layers[0][:8]]
            shared = tuple(t.cpu().numpy() for t in layers[0][8])
            hx, hr = x.float().cpu().numpy(), rw.cpu().numpy()
            if ref8 is not None:
                moe_kind = "reference"
                tabs = [np.array([e[k].ctypes.data for e in routed], dtype=np.uint64) for k in range(6)]
                out_r, out_s = np.empty((1, 7168), dtype=np.float32), np.empty((1, 7168), dtype=np.float32)

                def ref_moe():
                    ref8.fp8_e4m3_block_mlp_many_weighted_f32(*[t.ctypes.data for t in tabs], hx.ctypes.data,
                                                              hr.ctypes.data, out_r.ctypes.data, 8, 1, 2048, 7168, 56, 16)
                    ref8.fp8_e4m3_block_mlp_f32(*[t.ctypes.data for t in shared], hx.ctypes.data, out_s.ctypes.data,
                                                1, 2048, 7168, 56, 16)

                cpu_us = cpu_time(ref_moe)
                omp.omp_set_num_threads(1)
                cpu1_us = cpu_time(ref_moe)
                omp.omp_set_num_threads(all_threads)
            else:
                cpu_us = cpu_time(lambda: (oracle.fp8_mlp_many_weighted(routed, hx, hr), oracle.fp8_mlp(*shared, hx)))
            cpu_gbs = nbytes / (cpu_us / 1e6) / 1e9
            del routed, shared
        rows_out.append(("ds-v3 MoE layer (8 routed + shared, 2 launches)", 1, 1e3 * med, gbs, 100 * gbs / PEAK_HBM_GBS,
                         cpu_us, cpu_gbs, moe_kind, cpu1_us))
        rows_out.append((dev_name, 1, 1e3 * dev_med, dev_gbs, 100 * dev_gbs / PEAK_HBM_GBS, cpu_us, cpu_gbs, moe_kind,
                         cpu1_us))
        for name, us in decode_steps(layers, dev_tables, logits, x):
            gbs_s = nbytes / (us / 1e6) / 1e9
            rows_out.append((name, 1, us, gbs_s, 100 * gbs_s / PEAK_HBM_GBS, None, None, "port", None))
        del layers, dev_tables
        torch.cuda.empty_cache()

    def decode_steps(layers, dev_tables, logits, x):
        """Whole decode steps, router included, by wall clock over 30 steps:
        the reference's order (route, read the indices on the host, launch the
        chosen experts), the device-routed step, and that step replayed as one
        HIP graph."""
        k = 8
        route_w = torch.empty((1, k), device="cuda")
        yb = torch.empty((1, 7168), dtype=torch.bfloat16, device="cuda")
        y2 = torch.empty((1, 7168), device="cuda")
        ys2 = torch.empty((1, 7168), device="cuda")
        rej = torch.zeros((1,), dtype=torch.int32, device="cuda")
        idx0, _w0 = native.route_deepseek(logits)
        slot = {e: j for j, e in enumerate(idx0[0].tolist())}  # expert id -> the layer's j-th expert

        def host_step(i):
            idx, w = native.route_deepseek(logits)
            chosen = sorted(idx[0].tolist())  # the host read-back
            order = [slot[e] for e in chosen]
            layer = layers[i % len(layers)]
            tabs = [(ctypes.c_uint64 * 9)(*([layer[j][r].data_ptr() for j in order] + [layer[8][r].data_ptr()]))
                    for r in range(6)]
            pos = {e: j for j, e in enumerate(idx[0].tolist())}
            route_w.copy_(w[0, [pos[e] for e in chosen]].float().reshape(1, k))
            lib.pocketlm_set_stream(_stream_ptr(torch))
            rc = lib.fp8_e4m3_block_mlp_many_weighted_shared_bf16x_f32(
                *[ctypes.cast(t, ctypes.c_void_p) for t in tabs], ctypes.c_void_p(x.data_ptr()),
                ctypes.c_void_p(route_w.data_ptr()), ctypes.c_void_p(y2.data_ptr()), ctypes.c_void_p(ys2.data_ptr()),
                k, 1, 2048, 7168, 56, 16)
            if rc != 0:
                raise RuntimeError("host-routed step failed")
            torch.add(y2.to(torch.bfloat16), ys2.to(torch.bfloat16), out=yb)

        def dev_step(i):
            idx, w = native.route_deepseek(logits, weights_dtype=torch.float32)
            t = dev_tables[i % len(dev_tables)]
            lib.pocketlm_set_stream(_stream_ptr(torch))
            rc = lib.fp8_e4m3_block_moe_device_routed_bf16x_f32(
                ctypes.c_void_p(t[0].data_ptr()), 256, ctypes.c_void_p(idx.data_ptr()),
                ctypes.c_void_p(w.data_ptr()), k, ctypes.cast(t[1], ctypes.c_void_p),
                ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y2.data_ptr()), ctypes.c_void_p(ys2.data_ptr()),
                ctypes.c_void_p(yb.data_ptr()), ctypes.c_void_p(rej.data_ptr()), 1, 2048, 7168, 56, 16)
            if rc != 0:
                raise RuntimeError("device-routed step failed")

        def wall(fn, n=30):
            for i in range(3):
                fn(i)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for i in range(n):
                fn(i)
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) / n * 1e6

        out = [("ds-v3 router + MoE step, host read-back (reference order)", wall(host_step)),
               ("ds-v3 router + MoE step, device-routed", wall(dev_step))]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graphs = []
        with torch.cuda.stream(side):
            for i in range(len(dev_tables)):
                dev_step(i)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        for i in range(len(dev_tables)):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                dev_step(i)
            graphs.append(g)
        out.append(("ds-v3 router + MoE step, device-routed, one HIP graph", wall(lambda i: graphs[i % len(graphs)].replay())))
        # four steps per graph: the runtime's gap between back-to-back graph
        # launches (about 9 us in a kernel trace) is paid once per four steps
        graphs4 = []
        for j in range(2):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                for i in range(4):
                    dev_step(4 * j + i)
            graphs4.append(g)
        out.append(("ds-v3 router + MoE step, device-routed, 4 steps per HIP graph",
                    wall(lambda i: graphs4[i % 2].replay(), n=10) / 4))
        lib.pocketlm_set_stream(_stream_ptr(torch))
        for name, us in out:
            print(f"{name:40s} M=1  {us:9.2f} us (wall clock per step)", flush=True)
        return out

    if want("ds-v3 MoE layer"):
        moe_layer()

    def lm_head(vocab, hid, label):
        # vocabulary x hidden bf16 weight (over 1 GB: no copy rotation needed), top 50
        w = (torch.randn((vocab, hid), generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
        h = torch.randn((hid,), generator=gen, device="cuda").to(torch.bfloat16)
        ids = torch.empty((50,), dtype=torch.int64, device="cuda")
        lg = torch.empty((50,), device="cuda")
        lib.pocketlm_set_stream(_stream_ptr(torch))
        call = lambda: lib.native_lm_head_topk_u16(ctypes.c_void_p(h.data_ptr()), ctypes.c_void_p(w.data_ptr()),
                                                   ctypes.c_void_p(ids.data_ptr()), ctypes.c_void_p(lg.data_ptr()),
                                                   vocab, hid, 50, 1, 0)
        measure(f"lm_head top-50 {label} {vocab}x{hid} (bf16)", 1, lambda: [call], vocab * hid * 2 + hid * 2 + 50 * 12)
        del w

    if want("lm_head"):
        lm_head(152064, 3584, "Qwen2.5-7B")
        lm_head(129280, 7168, "DeepSeek-V3")
        torch.cuda.empty_cache()

    def dense_layer(ctx_len):
        # One Qwen2.5-7B decoder layer decode (fp16, row8-packed weights
        # N(0, 0.02), q/k/v biases) over a ctx_len-row KV cache; the new row
        # is rolled back after each call so every call sees ctx_len + 1 rows.
        # Two copies of the weights alternate so that the 466 MB do not stay
        # in the last-level cache.
        H, I, nh, nkv = 3584, 18944, 28, 4
        kvw = H // nh * nkv
        shapes = [(H, H), (kvw, H), (kvw, H), (H, H), (I, H), (I, H), (H, I)]
        sets = []
        for _ in range(2):
            sets.append([native.pack_weight_rows8((torch.randn(s, generator=gen, device="cuda") * 0.02).half())
                         for s in shapes])
        torch.cuda.empty_cache()
        norms = [(torch.rand(H, generator=gen, device="cuda") + 0.5).half() for _ in range(2)]
        biases = [(torch.randn(n, generator=gen, device="cuda") * 0.1).half() for n in (H, kvw, kvw)]
        hid = torch.randn(H, generator=gen, device="cuda").half()
        out = torch.empty(H, dtype=torch.float16, device="cuda")
        sess = lib.kv_prefill_init_typed(1, ctx_len + 8, kvw, 0)
        kv = torch.randn((2, ctx_len, kvw), generator=gen, device="cuda").half()
        lib.pocketlm_set_stream(_stream_ptr(torch))
        assert lib.kv_append_committed(sess, 0, kv[0].data_ptr(), kv[1].data_ptr(), ctx_len) == 0
        p = lambda t: t.data_ptr()  # noqa: E731

        def call_for(ws):
            args = [sess, 0, p(hid), p(norms[0]), p(norms[1]), *[p(w) for w in ws], *[p(b) for b in biases], None,
                    None, p(out), H, I, nh, nkv, 1e-6, 1e6]
            return lambda: lib.kv_dense_layer_decode_u16_ext_packed_rows8(*args) or lib.kv_rollback(sess)

        nbytes = sum(a * b for a, b in shapes) * 2 + 2 * (ctx_len + 1) * kvw * 2 + 8 * H * 2
        measure(f"dense decode layer Qwen2.5-7B, {ctx_len}-row KV cache (fp16 row8)", 1,
                lambda: [call_for(ws) for ws in sets], nbytes)
        torch.cuda.synchronize()
        lib.kv_free(sess)
        del sets
        torch.cuda.empty_cache()

    if want("dense decode layer"):
        dense_layer(1024)
        dense_layer(8192)

    def mla_flash(cache_len):
        # DeepSeek-V3 MLA attention of one token: 128 heads, nope 128, rope 64,
        # latent rank 512, v 128; fp32 wkv_b [128, 256, 512] (67 MB) in six
        # copies (402 MB, more than the memory-side cache holds), a
        # cache_len-row latent cache (fp32, as the reference keeps it)
        H, nope, rope, R, v = 128, 128, 64, 512, 128
        qn = torch.randn((H, nope), generator=gen, device="cuda") * 0.05
        qp = torch.randn((H, rope), generator=gen, device="cuda") * 0.05
        kvc = torch.randn((cache_len, R), generator=gen, device="cuda")
        pec = torch.randn((cache_len, rope), generator=gen, device="cuda")
        ws = [torch.randn((H, nope + v, R), generator=gen, device="cuda") * 0.02 for _ in range(6)]
        out = torch.empty((H, v), device="cuda")
        lib.pocketlm_set_stream(_stream_ptr(torch))
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        calls = [lambda w=w: lib.ds_mla_attention_flash_forward(p(qn), p(qp), p(kvc), p(pec), p(w), p(out), H, cache_len,
                                                                nope, rope, R, v, 1.0 / math.sqrt(192.0)) for w in ws]
        nbytes = H * (nope + v) * R * 4 + cache_len * (R + rope) * 4 + H * (nope + rope) * 4 + H * v * 4
        host = [t.cpu().numpy() for t in (qn, qp, kvc, pec, ws[0])]

        def cpu_mla():  # the reference's own formulation (native/__init__.py:857-876), numpy float64
            oracle_mla.mla_flash_closed_form(*host, 1.0 / math.sqrt(192.0))

        measure(f"mla attention DeepSeek-V3, {cache_len}-row latent cache (fp32)", 1, lambda: calls, nbytes,
                cpu_fn=cpu_mla)
        del ws
        torch.cuda.empty_cache()

    if want("mla attention"):
        mla_flash(1024)
        mla_flash(4096)

    def mla_block(prev_len):
        # DeepSeek-V3 attention block of one token with fp32 weights (the
        # reference's ds_attention_block_forward_f32): q_a 1536x7168, q_b
        # 24576x1536, kv_a 576x7168, kv_b 32768x512, o 7168x16384 (750 MB)
        hid, qr, R, H, nope, rope, v = 7168, 1536, 512, 128, 128, 64, 128
        w = [torch.randn(s, generator=gen, device="cuda") * 0.02
             for s in ((qr, hid), (H * (nope + rope), qr), (R + rope, hid), (H * (nope + v), R), (hid, H * v))]
        norms = [torch.ones(qr, device="cuda"), torch.ones(R, device="cuda")]
        x = torch.randn(hid, generator=gen, device="cuda")
        kvb = torch.randn((prev_len + 1, R), generator=gen, device="cuda")
        peb = torch.randn((prev_len + 1, rope), generator=gen, device="cuda")
        cs = [torch.ones(rope // 2, device="cuda"), torch.zeros(rope // 2, device="cuda")]
        out = torch.empty(hid, device="cuda")
        sess = lib.ds_session_create(1, hid, 0, 0, None, None)
        lib.pocketlm_set_stream(_stream_ptr(torch))
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        call = lambda: lib.ds_attention_block_forward_f32(sess, p(x), *[p(t) for t in w], *[p(t) for t in norms],  # noqa: E731
                                                          p(kvb), p(peb), *[p(t) for t in cs], p(kvb), p(peb), p(out),
                                                          hid, qr, R, H, nope, rope, v, prev_len, 1e-6,
                                                          1.0 / math.sqrt(192.0))
        nbytes = sum(t.numel() for t in w) * 4 + (prev_len + 1) * (R + rope) * 4 + 2 * hid * 4
        measure(f"ds-v3 attention block, {prev_len}-row latent cache (fp32 weights)", 1, lambda: [call], nbytes)
        torch.cuda.synchronize()
        lib.ds_session_destroy(sess)
        del w
        torch.cuda.empty_cache()

    def mla_fp8_block(prev_len):
        # The FP8 model's one-token attention (fp8_source.py:6337-6454) at
        # DeepSeek-V3 shapes: FP8 q_a 1536x7168, q_b 24576x1536, kv_a 576x7168,
        # o 7168x16384 (170 MB with scales), kv_b dequantized fp32 32768x512
        # (67 MB), bf16 hidden state; two weight sets rotated
        hid, qr, R, H, nope, rope, v = 7168, 1536, 512, 128, 128, 64, 128
        shapes = {"q_a": (qr, hid), "q_b": (H * (nope + rope), qr), "kv_a": (R + rope, hid), "o": (hid, H * v)}
        sets = []
        for _ in range(2):
            fp8 = {}
            for k, (rows, cols) in shapes.items():
                w = torch.randn((rows, cols), generator=gen, device="cuda").mul_(0.02).to(torch.float8_e4m3fn)
                s = torch.rand((math.ceil(rows / 128), math.ceil(cols / 128)), generator=gen, device="cuda") + 0.5
                fp8[k] = (w.view(torch.uint8), s)
            kvb = torch.randn((H * (nope + v), R), generator=gen, device="cuda") * 0.02
            sets.append((fp8, kvb))
        norms = [torch.ones(qr, device="cuda"), torch.ones(R, device="cuda")]
        x = torch.randn(hid, generator=gen, device="cuda").to(torch.bfloat16)
        kvc = torch.randn((prev_len + 1, R), generator=gen, device="cuda")
        pec = torch.randn((prev_len + 1, rope), generator=gen, device="cuda")
        cs = [torch.ones(rope // 2, device="cuda"), torch.zeros(rope // 2, device="cuda")]
        out = torch.empty(hid, device="cuda")
        lib.pocketlm_set_stream(_stream_ptr(torch))
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

        def call(fp8, kvb):
            return lib.ds_fp8_attention_block_bf16x_f32(
                p(x), *[p(t) for k in ("q_a", "q_b", "kv_a") for t in fp8[k]], p(kvb), *[p(t) for t in fp8["o"]],
                *[p(t) for t in norms], p(kvc), p(pec), *[p(t) for t in cs], p(kvc), p(pec), p(out), hid, qr, R, H,
                nope, rope, v, prev_len, 1e-6, 1.0 / math.sqrt(192.0))

        calls = [lambda st=st: call(*st) for st in sets]
        fp8_bytes = sum(r * c + 4 * math.ceil(r / 128) * math.ceil(c / 128) for r, c in shapes.values())
        nbytes = fp8_bytes + H * (nope + v) * R * 4 + (prev_len + 1) * (R + rope) * 4 + 2 * hid + 4 * hid
        measure(f"ds-v3 attention block, {prev_len}-row latent cache (FP8 weights, fp32 kv_b)", 1, lambda: calls,
                nbytes)
        del sets
        torch.cuda.empty_cache()

    if want("attention block"):
        mla_block(4096)
        mla_fp8_block(4096)

    transfers = []
    if want("fp8 pack -> HBM"):
        transfers.append(pack_transfer(torch))

    lines = [f"CPU: the reference's own fp8_linear.cpp / fp16_packed_gemv.cpp built from its sources "
             f"(oracle/_ref, kind \"reference\"; FP8 batches in its default mode, one weight pass per row, "
             f"which outran its one-pass batch mode here) with {all_threads} "
             "OpenMP threads and with one, else the oracle's restatement (kind \"port\"); weights warm in "
             "host RAM; about 1.5 s of calls per figure.", "",
             "| workload | M | GPU µs (mean) | GPU GB/s | % of 8 TB/s | CPU µs | CPU GB/s | CPU kind | CPU 1-thread µs |",
             "|---|---|---|---|---|---|---|---|---|"]
    for name, m, us, gbs, pct, cus, cgbs, kind, c1 in rows_out:
        lines.append(f"| {name} | {m} | {us:.2f} | {gbs:.0f} | {pct:.1f} | "
                     + (f"{cus:.0f} | {cgbs:.2f} | {kind} | " if cus else "— | — | — | ")
                     + (f"{c1:.0f} |" if c1 else "— |"))
    if transfers:
        lines += ["", "Weight files to HBM (file in the page cache, median of 5 loads; PCIe 5.0 x16 = 64 GB/s "
                  "per direction):", "",
                  "| transfer | MB | ms | GB/s | % of 64 GB/s | mmap + torch .to(device) ms | its GB/s |",
                  "|---|---|---|---|---|---|---|"]
        for name, nbytes, ms, base_ms in transfers:
            lines.append(f"| {name} | {nbytes / 1e6:.1f} | {ms:.1f} | {nbytes / ms / 1e6:.1f} | "
                         f"{100 * nbytes / ms / 1e6 / 64:.1f} | {base_ms:.1f} | {nbytes / base_ms / 1e6:.1f} |")
    text = "\n".join(lines)
    print(text)
    if args.table_out:
        Path(args.table_out).write_text(text + "\n")


def pack_transfer(torch):
    """One DeepSeek-V3 layer's 8 routed experts (352.5 MB) written as an FP8
    pack and loaded into HBM by layer and expert id through the native
    staging pipeline, against the host path of the reference's reader (mmap
    views, torch.frombuffer, .to(device) per tensor)."""
    import shutil
    import tempfile

    from pocketlm_amd import packs

    gen = torch.Generator().manual_seed(7)
    tensors = {}
    for e in range(8):
        for proj, shape in (("gate_proj", (2048, 7168)), ("up_proj", (2048, 7168)), ("down_proj", (7168, 2048))):
            name = f"model.layers.5.mlp.experts.{e}.{proj}.weight"
            tensors[name] = torch.randint(0, 255, shape, dtype=torch.uint8, generator=gen)
            tensors[name + "_scale_inv"] = torch.rand(((shape[0] + 127) // 128, (shape[1] + 127) // 128), generator=gen)
    nbytes = sum(t.numel() * t.element_size() for t in tensors.values())
    root = Path(tempfile.mkdtemp(prefix="pack_bench_"))
    try:
        packs.write_fp8_pack(tensors, root / "model" / "artifacts" / "fp8_pack", pack_bytes=1 << 30)
        del tensors
        reader = packs.FP8PackReader(root / "model")
        ids = list(range(8))
        names = [n for n in reader.tensors]

        def native_load():
            return reader.load_layer_experts(5, ids)

        def torch_load():
            out = {}
            for n in names:
                view = reader.get_tensor_bytes(n)
                out[n] = torch.frombuffer(view, dtype=torch.uint8).to("cuda")
                del view
            return out

        times = {}
        for label, fn in (("native", native_load), ("torch", torch_load)):
            fn()
            torch.cuda.synchronize()
            runs = []
            for _ in range(5):
                t0 = time.perf_counter()
                res = fn()
                torch.cuda.synchronize()
                runs.append((time.perf_counter() - t0) * 1e3)
                del res
            times[label] = sorted(runs)[2]
        reader.close()
    finally:
        shutil.rmtree(root, ignore_errors=True)
    name = "fp8 pack -> HBM, 8 DS-V3 experts"
    print(f"{name:40s} {nbytes / 1e6:.1f} MB  {times['native']:.1f} ms  {nbytes / times['native'] / 1e6:.1f} GB/s  "
          f"(mmap + torch .to(device): {times['torch']:.1f} ms)", flush=True)
    return name, nbytes, times["native"], times["torch"]


def pmc_probe(args):
    """Counter calibration workload: bench_moe_layer with 2 warm-up and 10
    timed steps (12 fused steps, 10 MoE-only calls, 10 router + MoE pairs),
    then 3 copies of a 256 MiB fp32 buffer (256 MiB read + 256 MiB written
    per copy).  The copy's FETCH_SIZE / WRITE_SIZE readings give the factor
    that turns the counters into bytes."""
    import torch

    from pocketlm_amd import _lib

    torch.cuda.set_device(0)
    lib = _lib.load()
    timer = Timer(torch)
    bench_moe_layer(torch, lib, timer, 10, 2)
    torch.cuda.synchronize()
    src = torch.ones(64 << 20, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("pmc probe done: 12 fused steps, 10 + 10 MoE layer calls, 3 copies of 268435456 bytes", flush=True)


def main(argv=None):
    args = _args(argv)
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2
    if str(REPO) not in sys.path:
        sys.path.insert(0, str(REPO))
    if args.table:
        table(args)
    elif args.pmc_probe:
        pmc_probe(args)
    else:
        main_line(args)
    return 0


if __name__ == "__main__":
    sys.exit(main())
