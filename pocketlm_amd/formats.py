"""Weight formats of the hot path, as torch code that runs on any device.

* Q4 (src/pcketlm/core/model_import/q4_quantize.py:21-91, scheme
  ``per-channel-symmetric-v1`` in q4_plan.py:13-14): one fp16 scale per
  output row (max|row| / 7, 1 for an all-zero row), values rounded half to
  even and clamped to [-7, 7], two's-complement nibbles flat over the whole
  tensor with element 2i in the low nibble of byte i.
* row8 (tools/pack_weights_row8.py:17-48): packed[blk, k, lane] =
  W[8*blk + lane, k], rows past the end zero.
* FP8 e4m3 with 128 x 128 block ``scale_inv`` (DeepSeek-V3): raw bytes plus
  an fp32 grid [ceil(rows/128), ceil(cols/128)].

These produce the inputs of the device kernels; the pack of a large weight
goes through the device kernel (``native.pack_weight_rows8``).
"""

from __future__ import annotations

import math

import torch

Q4_FORMAT = "pcketlm-q4"
Q4_SCHEME = "per-channel-symmetric-v1"
ROW_BLOCK = 8


def pack_int4(values: torch.Tensor) -> torch.Tensor:
    """Pack signed int4 values in [-8, 7] two per byte (element 2i low)."""
    flat = values.detach().to(torch.int16).flatten()
    if flat.numel() == 0:
        return torch.empty((0,), dtype=torch.uint8, device=values.device)
    if int(flat.min().item()) < -8 or int(flat.max().item()) > 7:
        raise ValueError("int4 values must be in the range [-8, 7].")
    enc = torch.bitwise_and(flat, 0x0F).to(torch.uint8)
    if enc.numel() % 2:
        enc = torch.cat([enc, torch.zeros((1,), dtype=torch.uint8, device=enc.device)])
    return torch.bitwise_or(enc[0::2], torch.bitwise_left_shift(enc[1::2], 4)).contiguous()


def unpack_int4(packed: torch.Tensor, value_count: int) -> torch.Tensor:
    """Inverse of pack_int4 (int8 values)."""
    b = packed.detach().to(torch.uint8).flatten()
    u = torch.empty((b.numel() * 2,), dtype=torch.int16, device=b.device)
    u[0::2] = torch.bitwise_and(b, 0x0F).to(torch.int16)
    u[1::2] = torch.bitwise_and(torch.bitwise_right_shift(b, 4), 0x0F).to(torch.int16)
    return torch.where(u >= 8, u - 16, u)[: int(value_count)].to(torch.int8).contiguous()


def _rows_view(t: torch.Tensor) -> torch.Tensor:
    if t.ndim == 0:
        return t.reshape(1, 1)
    if t.ndim == 1:
        return t.reshape(t.shape[0], 1)
    return t.reshape(t.shape[0], -1)


def quantize_tensor_to_q4(tensor: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, dict]:
    """Per-row symmetric Q4 of ``tensor`` on its own device.

    Returns (packed uint8 [ceil(numel/2)], scales fp16 [rows], metadata).
    """
    shape = [int(v) for v in tensor.shape]
    work = tensor.detach().float()
    m = _rows_view(work)
    max_abs = m.abs().amax(dim=1)
    # The two divisions are those of the reference's fp32 torch code on the
    # CPU, correctly rounded.  A GPU's fp32 division need not be (one ulp
    # moves a quotient across a .5 and changes the nibble), so they are done
    # in fp64 and rounded to fp32: for fp32 operands that gives the correctly
    # rounded fp32 quotient (53 >= 2 * 24 + 2 bits: no double-rounding error).
    scales = torch.where(max_abs > 0, (max_abs.double() / 7.0).float(), torch.ones_like(max_abs))
    q = torch.round((m.double() / scales.double()[:, None]).float()).clamp(-7, 7).to(torch.int8)
    packed = pack_int4(q.flatten())
    scale_tensor = scales.to(torch.float16).contiguous()
    meta = {
        "shape": shape,
        "scheme": Q4_SCHEME,
        "numel": int(work.numel()),
        "packed_numel": int(packed.numel()),
        "scale_shape": [int(v) for v in scale_tensor.shape],
    }
    return packed, scale_tensor, meta


def dequantize_q4_tensor(packed: torch.Tensor, scales: torch.Tensor, shape: list[int], *,
                         dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """torch form of the Q4 dequant (q4_quantize.py:74-91)."""
    count = int(math.prod(shape)) if shape else 1
    q = unpack_int4(packed, count).to(torch.float32)
    restored = _rows_view(q.reshape(shape) if shape else q.reshape(())) * scales.detach().float().reshape(-1, 1)
    return restored.reshape(shape).to(dtype=dtype).contiguous()


def q4_dequant_shape_params(shape: list[int]) -> tuple[int, int]:
    """(num_channels, channel_size) for a Q4 tensor (tensor_loader.py:598-605)."""
    if not shape:
        return 1, 1
    count = int(math.prod(shape))
    if len(shape) == 1:
        return int(shape[0]), 1
    return int(shape[0]), max(1, count // int(shape[0]))


def pack_rows8_tensor(tensor: torch.Tensor) -> torch.Tensor:
    """row8 interleave of a 2-D fp16/bf16 tensor, as uint16, on its own device."""
    if tensor.dtype not in {torch.float16, torch.bfloat16}:
        raise TypeError("row8 packing requires torch.float16 or torch.bfloat16 tensors")
    if tensor.ndim != 2:
        raise ValueError("row8 packing requires a 2D tensor")
    rows, cols = int(tensor.shape[0]), int(tensor.shape[1])
    blocks = (rows + ROW_BLOCK - 1) // ROW_BLOCK
    src = tensor.detach().contiguous().view(torch.uint16)
    padded = torch.zeros((blocks * ROW_BLOCK, cols), dtype=torch.uint16, device=src.device)
    padded[:rows] = src
    return padded.reshape(blocks, ROW_BLOCK, cols).transpose(1, 2).contiguous().reshape(-1)


def unpack_rows8_tensor(packed: torch.Tensor, rows: int, cols: int, *, dtype: torch.dtype) -> torch.Tensor:
    """Inverse of pack_rows8_tensor."""
    if dtype not in {torch.float16, torch.bfloat16}:
        raise TypeError("row8 unpack requires torch.float16 or torch.bfloat16 dtype")
    blocks = (int(rows) + ROW_BLOCK - 1) // ROW_BLOCK
    view = packed.detach().contiguous().view(torch.uint16).reshape(blocks, int(cols), ROW_BLOCK)
    return view.transpose(1, 2).reshape(blocks * ROW_BLOCK, int(cols))[: int(rows)].contiguous().view(dtype)


def fp8_e4m3_block_quantize(weight: torch.Tensor, *, block: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """Block-scaled e4m3 quantization of a 2-D weight (amax / 448 per block):
    returns (uint8 bytes, fp32 scale_inv grid) in the DeepSeek-V3 layout."""
    rows, cols = int(weight.shape[0]), int(weight.shape[1])
    br, bc = (rows + block - 1) // block, (cols + block - 1) // block
    w = torch.zeros((br * block, bc * block), dtype=torch.float32, device=weight.device)
    w[:rows, :cols] = weight.float()
    tiles = w.reshape(br, block, bc, block)
    amax = tiles.abs().amax(dim=(1, 3)).clamp_min(1e-12)
    scale = amax / 448.0
    q = (tiles / scale[:, None, :, None]).to(torch.float8_e4m3fn)
    data = q.reshape(br * block, bc * block)[:rows, :cols].contiguous().view(torch.uint8)
    return data, scale.float().contiguous()
