"""lm_head top-k on the GPU (native_lm_head_topk_u16, fp16_matmul.cpp:155-204):
the reference's own test (tests/test_native_fp16_matmul.py:75-86, against
torch.mv and torch.topk), vocabulary-sized weights, ties, fewer rows than
top_k, NaN rows and the one-thread-per-row path for odd sizes."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nat():
    from pocketlm_amd import native

    assert native.native_lm_head_topk_available(), "libpocketlm_hip.so must load on the GPU box"
    return native


def _want(weight, hidden, k, offset=0):
    logits = weight.float() @ hidden.float()
    vals, ids = torch.topk(logits, k)
    return vals, ids + offset


def test_reference_case_fp16_and_bf16(nat):
    torch.manual_seed(789)
    for dtype in (torch.float16, torch.bfloat16):
        hidden = (torch.randn((32,)) * 0.2).to(dtype)
        weight = (torch.randn((41, 32)) * 0.2).to(dtype)
        logits, ids = nat.lm_head_topk_u16(hidden.cuda(), weight.cuda(), top_k=5, token_offset=100)
        want_v, want_i = _want(weight, hidden, 5, 100)
        assert torch.equal(ids.cpu(), want_i.to(torch.int64))
        assert torch.allclose(logits.cpu(), want_v, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("rows,cols,k", [(150000, 512, 50), (40000, 7168, 64), (4097, 3584, 1)])
def test_vocabulary_sized_weights(nat, rows, cols, k):
    g = torch.Generator(device="cuda").manual_seed(rows)
    weight = (torch.randn((rows, cols), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    hidden = torch.randn((cols,), generator=g, device="cuda").to(torch.bfloat16)
    logits, ids = nat.lm_head_topk_u16(hidden, weight, top_k=k, token_offset=7)
    want_v, want_i = _want(weight, hidden, k, 7)
    assert torch.equal(ids, want_i)
    assert torch.allclose(logits, want_v, atol=1e-4, rtol=1e-5)
    assert bool((logits[:-1] >= logits[1:]).all())


def test_ties_short_vocabulary_nan_rows_and_odd_sizes(nat):
    g = torch.Generator().manual_seed(3)
    weight = (torch.randn((300, 64), generator=g) * 0.1).to(torch.float16)
    weight[[5, 40, 10, 250]] = weight[5] * 4  # four equal largest rows: 5, 10, 40, 250 in that order
    weight[7] = float("nan")
    hidden = torch.rand((64,), generator=g).to(torch.float16)
    logits, ids = nat.lm_head_topk_u16(hidden.cuda(), weight.cuda(), top_k=6)
    assert ids[:4].tolist() == [5, 10, 40, 250]
    assert 7 not in ids.tolist()
    # fewer rows than top_k: the rest is -1 / -inf
    logits3, ids3 = nat.lm_head_topk_u16(hidden.cuda(), weight[:3].cuda(), top_k=5)
    want_v, want_i = _want(weight[:3], hidden, 3)
    assert ids3[:3].tolist() == want_i.tolist() and ids3[3:].tolist() == [-1, -1]
    assert torch.isneginf(logits3[3:]).all()
    # an odd hidden size takes the one-thread-per-row kernel
    w_odd = (torch.randn((777, 33), generator=g) * 0.2).to(torch.bfloat16)
    h_odd = (torch.randn((33,), generator=g) * 0.2).to(torch.bfloat16)
    lo, io = nat.lm_head_topk_u16(h_odd.cuda(), w_odd.cuda(), top_k=9, token_offset=1000)
    want_v, want_i = _want(w_odd, h_odd, 9, 1000)
    assert io.cpu().tolist() == want_i.tolist()
    assert torch.allclose(lo.cpu(), want_v, atol=1e-5, rtol=1e-5)


def test_ties_across_selection_levels(nat):
    """Equal largest logits in different 1024-row blocks of the first
    selection level (and a second level over their survivors) come out in
    row order."""
    g = torch.Generator().manual_seed(8)
    weight = (torch.randn((70000, 64), generator=g) * 0.05).to(torch.bfloat16)
    top = weight[0] * 0 + 1.0
    for row in (66000, 100, 2000, 4500, 1024, 1023):
        weight[row] = top
    hidden = torch.rand((64,), generator=g).to(torch.bfloat16)
    logits, ids = nat.lm_head_topk_u16(hidden.cuda(), weight.cuda(), top_k=8, token_offset=5)
    assert ids[:6].tolist() == [r + 5 for r in (100, 1023, 1024, 2000, 4500, 66000)]
    assert len(set(logits[:6].tolist())) == 1 and logits[6] < logits[5]


def test_argument_errors(nat):
    w = torch.zeros((10, 16), dtype=torch.float16, device="cuda")
    h = torch.zeros((16,), dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="code 2"):
        nat.lm_head_topk_u16(h, w, top_k=65)
    with pytest.raises(TypeError):
        nat.lm_head_topk_u16(h.to(torch.bfloat16), w, top_k=2)
    with pytest.raises(ValueError):
        nat.lm_head_topk_u16(h[:8], w, top_k=2)
