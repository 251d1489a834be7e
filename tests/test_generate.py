"""The product decode scheduler (fdl.generate) against the literal restatement of the
reference loop (oracle/generate_oracle.py), step for step, on a tiny random model with
peaked logits (so multi-token acceptance, verify acceptance, EOS and refill all occur).
Both run the same unfused torch attention path on the CPU, so every decision must match
exactly: decoded token ids, token counts and per-prompt step counts."""
import numpy as np
import pytest
import torch

from fdl.generate import generate_with_Flash_dLLM, verify_mask
from fdl.model import LLaDAConfig, build_model
from fdl.torch_path import flash_fused_elastic_cache_torch
from oracle import flash_cache_oracle as orc
from oracle.generate_oracle import generate_oracle

TINY = dict(d_model=256, n_heads=2, n_layers=3, mlp_hidden_size=512, vocab_size=512,
            rope_theta=10000.0, mask_token_id=510, eos_token_id=509)


def _model(lm_head_std, seed=0):
    cfg = LLaDAConfig(**TINY, lm_head_std=lm_head_std)
    return build_model(cfg, flash_fused_elastic_cache_torch, "cpu", torch.float32, seed=seed)


def _prompts(n, lengths, vocab, seed):
    rng = np.random.default_rng(seed)
    out = []
    for L in lengths[:n]:
        p = rng.integers(0, vocab - 3, L)
        out.append(torch.from_numpy(p))
    return out


@pytest.mark.parametrize("verify", [False, True])
@pytest.mark.parametrize("lm_std,threshold,gamma,track,mask_num", [
    (1.0, 0.9, 0.9, 1, 1),    # peaked logits: several tokens per step, verify accepts
    (0.3, 0.7, 0.5, 2, 2),    # flatter: mostly one token per step, look-ahead window
    (0.8, 0.9, 0.9, -1, 1),   # track everything (full recompute every step)
])
def test_scheduler_matches_reference_loop(verify, lm_std, threshold, gamma, track, mask_num):
    model = _model(lm_std)
    lengths = [70, 96, 64]
    prompts = _prompts(3, lengths, TINY["vocab_size"], seed=1)
    kw = dict(gen_length=48, block_length=16, mask_id=510, threshold=threshold, gamma=gamma,
              track_num=track, mask_num=mask_num, eos_id=509, verify=verify)
    steps_o = [0] * 3
    resp_o, nt_o, mx_o = generate_oracle(model, prompts, lengths, 2, steps_o, **kw)
    steps_p = [0] * 3
    resp_p = [None] * 3
    resp_p, nt_p, mx_p = generate_with_Flash_dLLM(model, prompts, lengths, 2, resp_p, steps_p,
                                                  use_gpu_rank=False, rows_only=False, **kw)
    assert nt_p == nt_o and mx_p == mx_o
    assert steps_p == steps_o
    for i in range(3):
        assert resp_p[i] == resp_o[i], f"prompt {i}"
    assert max(steps_o) > 1


@pytest.mark.parametrize("verify", [False, True])
def test_scheduler_eos_and_verify_acceptance(verify):
    """EOS is set to the token the model emits most, so sequences end early and the
    predicted-length masking paths run; the verify pass accepts drafts."""
    from fdl.generate import DecodeStats
    model = _model(1.0, seed=3)
    lengths = [64, 72, 80]
    prompts = _prompts(3, lengths, TINY["vocab_size"], seed=4)
    kw = dict(gen_length=48, block_length=16, mask_id=510, threshold=0.9, gamma=0.8,
              track_num=1, mask_num=2, verify=verify)
    probe, _, _ = generate_with_Flash_dLLM(model, prompts, lengths, 2, [None] * 3, [0] * 3,
                                           eos_id=509, use_gpu_rank=False, rows_only=False, **kw)
    counts = np.bincount(np.concatenate([np.asarray(r) for r in probe]))
    # the most frequent emitted tokens, as EOS; skip one for which the reference loop itself
    # fails (a sequence that never emits EOS runs into the EOS padding until its masked
    # block is cut short by the slot row end: generate.py:215/:235 shape mismatch)
    for eos in np.argsort(-counts, kind="stable")[:12]:
        eos = int(eos)
        steps_o = [0] * 3
        try:
            resp_o, nt_o, mx_o = generate_oracle(model, prompts, lengths, 2, steps_o, eos_id=eos, **kw)
        except RuntimeError as e:
            assert "shape mismatch" in str(e)
            continue
        if any(eos in resp_o[i] for i in range(3)):
            break
    else:
        pytest.fail("no EOS candidate gives a well-defined reference run that decodes EOS")
    st = DecodeStats()
    steps_p = [0] * 3
    resp_p, nt_p, mx_p = generate_with_Flash_dLLM(model, prompts, lengths, 2, [None] * 3, steps_p,
                                                  eos_id=eos, use_gpu_rank=False, rows_only=False,
                                                  stats=st, **kw)
    assert (nt_p, mx_p, steps_p) == (nt_o, mx_o, steps_o)
    assert resp_p == [resp_o[i] for i in range(3)]
    assert any(eos in r for r in resp_p)  # the EOS paths (predicted length) ran
    if verify:
        assert st.verify_accepted > 0


def test_scheduler_survives_reference_runaway_case():
    """The case where the reference loop fails (masked block cut short at the slot row end
    in verify mode) completes in the product scheduler with every sequence finished."""
    model = _model(1.0, seed=3)
    lengths = [64, 72, 80]
    prompts = _prompts(3, lengths, TINY["vocab_size"], seed=4)
    kw = dict(gen_length=48, block_length=16, mask_id=510, threshold=0.9, gamma=0.8,
              track_num=1, mask_num=2, verify=True, eos_id=52)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        generate_oracle(model, prompts, lengths, 2, [0] * 3, **kw)
    resp, nt, mx = generate_with_Flash_dLLM(model, prompts, lengths, 2, [None] * 3, [0] * 3,
                                            use_gpu_rank=False, rows_only=False, **kw)
    assert all(r is not None for r in resp) and nt >= 48 * 2


def test_scheduler_rows_only_equivalent():
    """LM head on the read rows only gives the same decisions (row-wise head)."""
    model = _model(1.0)
    lengths = [64, 80]
    prompts = _prompts(2, lengths, TINY["vocab_size"], seed=2)
    kw = dict(gen_length=32, block_length=16, mask_id=510, threshold=0.9, gamma=0.9,
              track_num=1, mask_num=1, eos_id=509, verify=True, use_gpu_rank=False)
    r1, n1, _ = generate_with_Flash_dLLM(model, prompts, lengths, 2, [None] * 2, [0] * 2, rows_only=True, **kw)
    r2, n2, _ = generate_with_Flash_dLLM(model, prompts, lengths, 2, [None] * 2, [0] * 2, rows_only=False, **kw)
    assert n1 == n2
    agree = np.mean([a == b for x, y in zip(r1, r2) for a, b in zip(x, y)])
    assert agree >= 0.99


@pytest.mark.parametrize("T,S", [(32, 0), (30, 1), (16, 8), (0, 16), (20, 6)])
def test_verify_mask_closed_form_matches_construction(T, S):
    bm = 16
    if T + 2 * S != 2 * bm:
        T = 2 * bm - 2 * S
    np.testing.assert_array_equal(verify_mask(T, S, bm), orc.verify_mask(T, S, bm))


def test_page_pool_alloc_free():
    from fdl.schedule import PagePool, page_slots
    pool = PagePool(10)
    a = pool.alloc(3)
    b = pool.alloc(4)
    assert a.tolist() == [0, 1, 2] and b.tolist() == [3, 4, 5, 6] and pool.n_free == 3
    pool.free(a)
    c = pool.alloc(5)  # lowest free ids, ascending
    assert c.tolist() == [0, 1, 2, 7, 8] and pool.n_free == 1
    with pytest.raises(MemoryError):
        pool.alloc(2)
    with pytest.raises(ValueError):
        pool.free(np.array([9]))  # never allocated
    pool.free(b)
    with pytest.raises(ValueError):
        pool.free(b)  # twice
    assert pool.pages_for(33) == 2 and pool.n_slots == 320
    s = page_slots(np.array([7, 2]), 40)
    assert s[:32].tolist() == list(range(224, 256)) and s[32:].tolist() == list(range(64, 72))


@pytest.mark.parametrize("eos", [509, 511])
@pytest.mark.parametrize("verify", [False, True])
def test_paged_pool_decode_matches_fixed_stride(verify, eos):
    """The decode over a paged K/V pool (pages handed out per sequence, grown, returned and
    reused on refill) gives the fixed-stride decode token for token when every row fits;
    with a pool too small for all rows at once, prompts wait for pages and still decode to
    the same tokens (each sequence's decode depends only on its own rows).
    Fixed stride: L = ((96 + 48 + 16) // 128 + 1) * 128 = 256 slots = 8 pages per row.
    Reservations max(seqlen_k, prompt + 48 + 15): 4, 8, 5, 8, 4 pages; prompt 79 starts with
    the 4 pages of its 128 keys. With EOS 511, which this model rarely emits, sequences
    decode past prompt + gen (as the reference loop does) and grow page by page beyond
    their reservation, up to the 8 pages of the stride."""
    model = _model(1.0, seed=6)
    lengths = [64, 96, 79, 80, 64]
    prompts = _prompts(5, lengths, TINY["vocab_size"], seed=8)
    kw = dict(gen_length=48, block_length=16, mask_id=510, threshold=0.9, gamma=0.9,
              track_num=1, mask_num=1, eos_id=eos, verify=verify, use_gpu_rank=False,
              rows_only=False)
    st = [0] * 5
    r0, n0, m0 = generate_with_Flash_dLLM(model, prompts, lengths, 3, [None] * 5, st, **kw)
    for pages, full in ((24, True),) + (((12, False),) if eos == 509 else ()):
        stp = [0] * 5
        r1, n1, m1 = generate_with_Flash_dLLM(model, prompts, lengths, 3, [None] * 5, stp,
                                              kv_pages=pages, **kw)
        assert r1 == r0 and n1 == n0 and m1 == m0, pages
        if full:
            assert stp == st
    with pytest.raises(MemoryError):
        generate_with_Flash_dLLM(model, prompts, lengths, 3, [None] * 5, [0] * 5, kv_pages=7, **kw)
