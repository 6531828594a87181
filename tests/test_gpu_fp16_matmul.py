"""fp16 matmul on the GPU (native_fp16_matmul, fp16_matmul.cpp:344-396): the
reference's own tests (tests/test_native_fp16_matmul.py:16-71: at most 1 fp16
ulp from the fp32 product rounded to fp16), larger ragged shapes, empty and
k = 0 shapes, integer-valued inputs whose fp32 sums are exact (bit-equal to
torch), and the argument codes."""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nat():
    from pocketlm_amd import native

    assert native.native_fp16_matmul_available(), "libpocketlm_hip.so must load on the GPU box"
    return native


def _ordered(t: torch.Tensor) -> torch.Tensor:
    bits = t.contiguous().view(torch.int16).to(torch.int32)
    return torch.where(bits < 0, 0x8000 - bits, bits)


def _max_ulp(a: torch.Tensor, b: torch.Tensor) -> int:
    return int((_ordered(a) - _ordered(b)).abs().max().item())


def _want(a, b):
    return (a.float() @ b.float()).to(torch.float16)


def test_reference_small_shapes(nat):
    torch.manual_seed(123)
    for m, k, n in [(1, 8, 8), (3, 9, 5), (8, 16, 8), (17, 31, 13)]:
        a = (torch.randn((m, k)) * 0.25).to(torch.float16)
        b = (torch.randn((k, n)) * 0.25).to(torch.float16)
        out = nat.fp16_matmul(a, b)
        assert out.dtype == torch.float16 and out.device.type == "cpu" and out.shape == (m, n)
        assert _max_ulp(out, _want(a, b)) <= 1


def test_reference_blas_switch_case(nat):
    torch.manual_seed(321)
    a = (torch.randn((5, 7)) * 0.2).to(torch.float16)
    b = (torch.randn((7, 3)) * 0.2).to(torch.float16)
    assert _max_ulp(nat.fp16_matmul(a, b), _want(a, b)) <= 1


@pytest.mark.parametrize("m,k,n", [(128, 128, 128), (70, 1000, 45), (1, 4096, 257), (300, 33, 1)])
def test_larger_ragged_shapes_on_device(nat, m, k, n):
    torch.manual_seed(m + k + n)
    a = torch.randn((m, k), dtype=torch.float16, device="cuda")
    b = torch.randn((k, n), dtype=torch.float16, device="cuda")
    out = nat.fp16_matmul(a, b)
    assert out.device.type == "cuda"
    ac, bc = a.cpu().double(), b.cpu().double()
    exact = ac @ bc
    # fp32 sums in any order are within k 2^-24 sum|a b| of the exact sum
    # (the standard summation error bound); rounding to fp16 adds half an ulp
    bound = k * 2.0 ** -24 * (ac.abs() @ bc.abs())
    half_ulp = torch.abs(exact.to(torch.float16).double()).clamp(min=2.0 ** -24) * 2.0 ** -11
    got = out.cpu().double()
    assert bool(((got - exact).abs() <= bound + 2 * half_ulp).all())
    # and mostly the same fp16 as torch's fp32 product
    same = (out.cpu() == _want(a.cpu(), b.cpu())).float().mean()
    assert float(same) > 0.95


def test_integer_inputs_are_exact(nat):
    # small integers: every product and partial sum is an exact fp32 integer
    g = torch.Generator().manual_seed(5)
    a = torch.randint(-8, 9, (37, 300), generator=g).to(torch.float16)
    b = torch.randint(-8, 9, (300, 29), generator=g).to(torch.float16)
    out = nat.fp16_matmul(a, b)
    assert torch.equal(out, (a.double() @ b.double()).to(torch.float16))


def test_empty_and_zero_k(nat):
    from pocketlm_amd import _lib

    lib = _lib.load()
    # m or n = 0 writes nothing; k = 0 writes zeros (the sgemm of an empty sum)
    c = torch.full((3, 5), 7.0, dtype=torch.float16, device="cuda")
    ab = torch.ones((16,), dtype=torch.float16, device="cuda")
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    assert lib.native_fp16_matmul(p(ab), p(ab), p(c), 0, 5, 4) == 0
    assert lib.native_fp16_matmul(p(ab), p(ab), p(c), 3, 0, 4) == 0
    torch.cuda.synchronize()
    assert bool((c == 7.0).all())
    assert lib.native_fp16_matmul(p(ab), p(ab), p(c), 3, 5, 0) == 0
    torch.cuda.synchronize()
    assert torch.equal(c.cpu(), torch.zeros((3, 5), dtype=torch.float16))
    # an empty tensor has no storage: the wrapper reports the null pointer, as the reference's does
    with pytest.raises(RuntimeError, match="code 1"):
        nat.fp16_matmul(torch.ones((0, 4), dtype=torch.float16), torch.ones((4, 3), dtype=torch.float16))


def test_argument_codes(nat):
    from pocketlm_amd import _lib

    lib = _lib.load()
    one = ctypes.c_void_p(16)
    assert lib.native_fp16_matmul(None, one, one, 1, 1, 1) == 1
    assert lib.native_fp16_matmul(one, one, one, -1, 1, 1) == 2
    assert lib.native_fp16_matmul(one, one, one, 1, 1, -1) == 2
    assert lib.native_fp16_matmul(one, one, one, 0, 5, 5) == 0
    with pytest.raises(TypeError):
        nat.fp16_matmul(torch.ones((2, 2)), torch.ones((2, 2)))
    with pytest.raises(ValueError):
        nat.fp16_matmul(torch.ones((2, 3), dtype=torch.float16), torch.ones((2, 3), dtype=torch.float16))
