"""LM-head confidence (fdl_softmax_confidence) against the float64 torch code it replaces
(generate.py:218, :320, :337): max(softmax(logits.double())) and its index, and the
softmax probability of a given token. The reference is torch's float64 softmax on the CPU:
the float64 terms are identical and only the order of the sum differs, so probabilities
agree to ~1e-13 relative and indices exactly. (torch's float64 softmax kernel on this ROCm
build is itself ~1e-9 off the CPU result, so it is not the reference here.)"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from fdl import ops

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("rows,vocab,std", [(1, 8, 1.0), (37, 126464, 0.02), (256, 126464, 3.0),
                                            (5, 4096, 30.0)])
def test_softmax_confidence_max_matches_torch_float64(rows, vocab, std):
    gen = torch.Generator().manual_seed(rows + vocab)
    logits = (torch.randn(rows, vocab, generator=gen) * std).to(torch.bfloat16)
    # ties at the maximum: the first index must win
    if vocab > 8:
        logits[0, 5] = logits[0, vocab - 3] = logits[0].max() + 1.0
    ref_p, ref_i = torch.max(F.softmax(logits.to(torch.float64), dim=-1), dim=-1)
    prob, arg = ops.softmax_confidence(logits.to(DEV))
    torch.cuda.synchronize()
    torch.testing.assert_close(prob.cpu(), ref_p, rtol=1e-12, atol=0)
    assert torch.equal(arg.cpu(), ref_i)
    if vocab > 8:
        assert int(arg[0]) == 5


def test_softmax_confidence_token_probability():
    gen = torch.Generator().manual_seed(7)
    rows, vocab = 40, 126464
    logits = (torch.randn(rows, vocab, generator=gen) * 2.0).to(torch.bfloat16)
    tok = torch.randint(0, vocab, (rows,), generator=gen)
    tok[3] = -1  # outside the vocabulary: probability 0
    ref = F.softmax(logits.to(torch.float64), dim=-1).gather(1, tok.clamp(min=0)[:, None]).view(-1)
    ref[3] = 0.0
    prob, _ = ops.softmax_confidence(logits.to(DEV), tok.to(DEV))
    torch.cuda.synchronize()
    torch.testing.assert_close(prob.cpu(), ref, rtol=1e-12, atol=1e-300)


def test_softmax_confidence_non_finite_rows_match_torch():
    """Rows of all -inf, with a NaN, with a +inf, and with the maximum tied at several
    places: the probability and index are torch.max(softmax(float64)) of the row (NaN and
    index 0 for the rows whose softmax is NaN; the first index of a tie)."""
    vocab = 1024
    x = torch.randn((5, vocab), generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    x[0] = float("-inf")
    x[1, 300] = float("nan")
    x[2, 700] = float("inf")
    x[3, 10] = x[3, 500] = x[3, 900] = 8.0  # tied maximum
    prob, arg = ops.softmax_confidence(x.to(DEV))
    ref_p, ref_i = torch.max(torch.softmax(x.double(), dim=-1), dim=-1)
    got_p, got_i = prob.cpu(), arg.cpu()
    assert torch.equal(got_i, ref_i), (got_i, ref_i)
    assert torch.isnan(got_p[:3]).all() and torch.isnan(ref_p[:3]).all()
    np.testing.assert_allclose(got_p[3:].numpy(), ref_p[3:].numpy(), rtol=1e-12)
