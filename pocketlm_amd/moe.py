"""DeepSeek MoE layer on the device: run_fp8_moe
(src/pcketlm/core/runtime/fp8_source.py:1569-1884) over this package's
native FP8 kernels, with the routed experts' weights resident in HBM.

The reference picks one of several paths, and so does this module, with the
same environment flags and the same bf16 accumulation:

* pair-weighted many-expert kernel, M > 1 and PCKETLM_ENABLE_FP8_MOE_PAIR_WEIGHTED_MANY
  (fp8_source.py:1647-1690);
* row-weighted many-expert kernel, M > 1 and PCKETLM_ENABLE_FP8_MOE_ROW_WEIGHTED_MANY,
  in chunks of PCKETLM_FP8_MOE_ROW_WEIGHTED_MANY_CHUNK experts (1691-1734);
* route-weighted many-expert kernel at M == 1 (1643-1646, 1736-1764);
* unweighted many-expert kernel at M == 1 when the weighted one is
  unavailable (1765-1800);
* otherwise one MLP per selected expert on the rows that chose it
  (1806-1836), accumulated in expert order as
  out[rows] += bf16(expert_out) * bf16(route).

The shared expert's MLP is added last (1838-1862); every add into the output
is a bf16 add.  Expert selection (sorted unique ids of the router's
indices) needs the indices on the host, as in the reference.

run_fp8_moe_device keeps the router's outputs on the device instead: the
experts are chosen on the device, in the gate/up launch, from a device
table of every expert (native.FP8ExpertTable), and the bf16 tail is done by the library, so the
layer issues no host read-back.  Its values are those of the weighted path
at M == 1 and of the row-weighted path at M > 1.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Mapping, Sequence

import torch

from . import native

__all__ = ["MoEOutput", "run_fp8_moe", "run_fp8_moe_device"]


def _enabled(name: str) -> bool:
    return os.environ.get(name, "").strip().lower() in {"1", "true", "yes", "on"}


def _row_chunk_size() -> int:
    raw = os.environ.get("PCKETLM_FP8_MOE_ROW_WEIGHTED_MANY_CHUNK", "").strip()
    try:
        return max(0, int(raw)) if raw else 0
    except ValueError:
        return 0


@dataclass
class MoEOutput:
    """Output of one MoE layer call (the tensor part of FP8MoEResult,
    fp8_source.py:312-354)."""

    output: torch.Tensor
    selected_experts: list[int]
    path: str


ExpertWeights = Sequence[torch.Tensor]  # gate, gate_scale_inv, up, up_scale_inv, down, down_scale_inv


def _same_shapes(a: ExpertWeights, b: ExpertWeights) -> bool:
    return all(tuple(ta.shape) == tuple(tb.shape) for ta, tb in zip(a, b))


def run_fp8_moe(hidden: torch.Tensor, route_indices: torch.Tensor, route_weights: torch.Tensor,
                experts: Mapping[int, ExpertWeights], shared: ExpertWeights | None = None, *,
                dtype: torch.dtype = torch.bfloat16) -> MoEOutput:
    """One DeepSeek MoE layer: routed experts chosen by the router plus the
    shared expert, output in ``dtype`` with the shape of ``hidden``.

    route_indices [M, k] int64 and route_weights [M, k] (the router's bf16
    weights) come from route_deepseek / run_fp8_router; experts maps an
    expert id to its six tensors (FP8 weights and fp32 scale_inv grids)."""
    flat = hidden.reshape(-1, hidden.shape[-1])
    m = int(flat.shape[0])
    idx = route_indices.reshape(m, -1)
    weights = route_weights.reshape(m, -1).float()
    selected = sorted({int(v) for v in idx.reshape(-1).tolist()})
    jobs = []
    for expert in selected:
        rows, tops = torch.where(idx == expert)
        if rows.numel():
            jobs.append((expert, rows, tops))
    missing = [e for e, _r, _t in jobs if e not in experts]
    if missing:
        raise KeyError(f"weights of selected experts {missing} were not provided")
    x = flat.to(dtype)
    out = torch.zeros_like(flat, dtype=dtype)
    items = [experts[e] for e, _r, _t in jobs]
    path = ""
    shared_out = None
    many_on = not _enabled("PCKETLM_DISABLE_NATIVE_FP8_MLP_MANY")

    if jobs and m > 1 and _enabled("PCKETLM_ENABLE_FP8_MOE_PAIR_WEIGHTED_MANY") \
            and native.native_fp8_mlp_many_pair_weighted_available():
        # (item, row, weight) pairs in expert order, rows ascending within an expert.
        pair_items = torch.cat([torch.full_like(rows, item) for item, (_e, rows, _t) in enumerate(jobs)])
        pair_rows = torch.cat([rows for _e, rows, _t in jobs])
        pair_w = torch.cat([weights[rows, tops] for _e, rows, tops in jobs])
        # The pairs come from the validated jobs, so the no-sync form (no host
        # read-back of the indices; same sums) is used.
        y, _bad = native.fp8_e4m3_block_mlp_many_pair_weighted_nosync(items, x, pair_items, pair_rows, pair_w)
        out += y.to(dtype)
        path = "pair_weighted"
    elif jobs and m > 1 and _enabled("PCKETLM_ENABLE_FP8_MOE_ROW_WEIGHTED_MANY") \
            and native.native_fp8_mlp_many_row_weighted_available():
        chunk = _row_chunk_size() or len(jobs)
        chunk = max(1, min(chunk, len(jobs)))
        total = torch.zeros((m, int(flat.shape[-1])), dtype=torch.float32, device=flat.device)
        for c0 in range(0, len(jobs), chunk):
            part = jobs[c0:c0 + chunk]
            route = torch.zeros((len(part), m), dtype=torch.float32, device=flat.device)
            for item, (_e, rows, tops) in enumerate(part):
                route[item, rows] = weights[rows, tops]
            total += native.fp8_e4m3_block_mlp_many_row_weighted_f32(items[c0:c0 + chunk], x, route)
        out += total.to(dtype)
        path = "row_weighted"
    elif jobs and m == 1 and many_on and native.native_fp8_mlp_many_weighted_available():
        route = torch.stack([weights[rows[0], tops[0]] for _e, rows, tops in jobs]).to(torch.float32)
        if shared is not None and len(items) < 64 and _same_shapes(items[0], shared):
            # routed and shared experts in the same two launches, same values
            y, shared_out = native.fp8_e4m3_block_mlp_many_weighted_shared_f32(items, shared, x, route)
        else:
            y = native.fp8_e4m3_block_mlp_many_weighted_f32(items, x, route)
        out += y.to(dtype)
        path = "weighted"
    else:
        if jobs and m == 1 and many_on and native.native_fp8_mlp_many_available():
            many = native.fp8_e4m3_block_mlp_many_f32(items, x)
            outs = [many[item, rows].to(dtype) for item, (_e, rows, _t) in enumerate(jobs)]
            path = "many"
        else:
            outs = [native.fp8_e4m3_block_mlp_f32(*experts[e], x[rows]).to(dtype) for e, rows, _t in jobs]
            path = "per_expert"
        for (_e, rows, tops), y in zip(jobs, outs):
            route = weights[rows, tops].view(-1, 1).to(dtype)
            out[rows] += y * route

    if shared is not None:
        if shared_out is None:
            shared_out = native.fp8_e4m3_block_mlp_f32(*shared, x)
        out = out + shared_out.to(dtype)
    return MoEOutput(output=out.reshape(hidden.shape).contiguous(), selected_experts=selected, path=path)


def run_fp8_moe_device(hidden: torch.Tensor, route_indices: torch.Tensor, route_weights: torch.Tensor,
                       table: "native.FP8ExpertTable", shared: ExpertWeights | None = None, *,
                       dtype: torch.dtype = torch.bfloat16) -> MoEOutput:
    """run_fp8_moe with the experts chosen on the device (no host read-back
    of the router's indices; at most 8 rows and 64 choices per call).

    table holds every routed expert of the layer; route_indices / route_weights
    are the router's [M, k] device tensors (route_deepseek; its
    weights_dtype=torch.float32 form skips two conversions).  selected_experts
    is left empty: reading it would need the host round trip this path avoids.
    """
    flat = hidden.reshape(-1, hidden.shape[-1])
    res = native.fp8_e4m3_block_moe_device_routed_f32(table, flat.to(dtype), route_indices, route_weights, shared,
                                                      bf16_output=dtype == torch.bfloat16)
    if res.output is not None:
        out = res.output
    else:
        out = torch.zeros_like(flat, dtype=dtype) + res.routed.to(dtype)
        if res.shared is not None:
            out = out + res.shared.to(dtype)
    return MoEOutput(output=out.reshape(hidden.shape).contiguous(), selected_experts=[], path="device_routed")
