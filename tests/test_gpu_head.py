"""LM-head confidence (fdl_softmax_confidence) against the float64 torch code it replaces
(generate.py:218, :320, :337): max(softmax(logits.double())) and its index, and the
softmax probability of a given token. The reference is torch's float64 softmax on the CPU:
the float64 terms are identical and only the order of the sum differs, so probabilities
agree to ~1e-13 relative and indices exactly. (torch's float64 softmax kernel on this ROCm
build is itself ~1e-9 off the CPU result, so it is not the reference here.)"""
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
