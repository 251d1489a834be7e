"""Known-answer tests of the decode loop (llada/generate.py:61-472), hand-worked.

A scripted model replaces the transformer: for every call it returns logits chosen per
(step, slot) — a row whose float64 softmax maximum is exactly the scripted confidence at
the scripted token — and writes scripted importance scores into attn_scores. The expected
decisions below are worked out by hand from the reference's rules, so these tests pin the
oracle's restatement (oracle/generate_oracle.py) independently of the product, and run the
product scheduler (fdl.generate) against the same answers.

Rules exercised (reference lines):
  pass-1 acceptance   keep = max(#(conf >= threshold), 1), confidences of slots at or past
                      the predicted length zeroed once EOS is decoded (:335-350)
  refresh order       decoded slots full_pos[:nd - keep] sorted ascending by score, ties
                      to the higher slot (the top of the order prefers lower slots) (:364-366)
  tracked set         full_pos[max(0, nd - track*bm) : nd] + full_pos[nd + bm :
                      min(k_end, nd + mask_num*bm)]; track < 0: every other slot (:367-381)
  verify lists        S = min(max(len - keep, 0), bm/2) candidates, T = 2bm - 2S fill rows
                      full_pos[nd - T : nd], rows [fill, draft(cand), mask(cand)], keys
                      full_pos[:nd - T] + full_pos[nd + S : k_end], the m11..m22 mask (:210-297)
  verify acceptance   keep = #(cumprod of the mask rows' draft-token probabilities >= gamma)
                      (:312-333)
  refill              a finished row takes the next prompt: x, k_end, nd, full_pos reset,
                      step-0 rows again (:405-427)
"""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from fdl.generate import generate_with_Flash_dLLM
from oracle.generate_oracle import generate_oracle

V, MASK, EOS = 16, 15, 14


def _row(tok: int, conf: float) -> torch.Tensor:
    """Logits whose float64 softmax has its maximum `conf` at `tok` (other entries 0)."""
    r = torch.zeros(V, dtype=torch.float32)
    r[tok] = float(np.log(conf * (V - 1) / (1.0 - conf)))
    return r


class Scripted:
    """Stands in for LLaDAModelLM: model(x_query, use_cache, lengths, positions).logits.

    script[step] = {"rows": {slot: (token, conf)}, "scores": {slot: value},
                    "verify_rows": {row index: (token, prob)}} for the step's calls (the
    first call of a step is the pass-1 forward, a verify forward is recognised by
    lengths[11]). `default` (token, conf) is used for pass-1 rows the script omits."""

    def __init__(self, script: dict, default=(3, 0.95)):
        self.config = SimpleNamespace(d_model=256, n_layers=2, n_heads=2, rope_theta=10000.0)
        self.device = torch.device("cpu")
        self.dtype = torch.float32
        self.model = SimpleNamespace(transformer=SimpleNamespace(blocks=[SimpleNamespace(), SimpleNamespace()]))
        self.script, self.default = script, default
        self.calls, self.step = [], -1

    def __call__(self, x_query, use_cache=True, lengths=None, positions=None):
        verify = bool(lengths[11])
        if not verify:
            self.step += 1
        qpos = positions[0].cpu().numpy().astype(np.int64).tolist()
        rec = {"step": self.step, "verify": verify, "qpos": qpos,
               "x": x_query.reshape(-1).cpu().numpy().tolist()}
        if verify:
            rec["keys"] = positions[1].cpu().numpy().astype(np.int64).tolist()
            rec["vblocks"] = np.asarray(lengths[1].cpu()).astype(np.int64).tolist()
            rec["mask"] = positions[5].cpu().numpy().astype(bool)
        else:
            rec["masked_blocks"] = np.asarray(lengths[2].cpu()).astype(np.int64).tolist()
            rec["tracked_blocks"] = np.asarray(lengths[3].cpu()).astype(np.int64).tolist()
        self.calls.append(rec)
        sc = self.script.get(self.step, {})
        logits = torch.zeros((len(qpos), V), dtype=torch.float32)
        if verify:
            for r, (tok, p) in sc.get("verify_rows", {}).items():
                logits[r] = _row(tok, p)
        else:
            rows = sc.get("rows", {})
            for r, s in enumerate(qpos):
                logits[r] = _row(*rows.get(s, self.default))
            for s, v in sc.get("scores", {}).items():
                positions[4][s] = v
        return SimpleNamespace(logits=logits[None])


def _run(impl, model, prompts, B, **kw):
    lengths = [len(p) for p in prompts]
    prompts = [torch.tensor(p, dtype=torch.int64) for p in prompts]
    n_steps = [0] * len(prompts)
    if impl == "oracle":
        resp, nt, mx = generate_oracle(model, prompts, lengths, B, n_steps, **kw)
        resp = [resp[i] for i in range(len(prompts))]
    else:
        resp, nt, mx = generate_with_Flash_dLLM(model, prompts, lengths, B, [None] * len(prompts),
                                               n_steps, use_gpu_rank=False, rows_only=False, **kw)
    return resp, nt, mx, n_steps


IMPLS = ["oracle", "product"]
P0 = [7, 8, 9, 10]  # a 4-token prompt


def _kw(**over):
    kw = dict(gen_length=8, block_length=4, mask_id=MASK, threshold=0.9, gamma=0.9,
              track_num=1, mask_num=1, eos_id=EOS, verify=False)
    kw.update(over)
    return kw


# Prompt of 4 tokens, gen 8, block 4: stride L = 128, k_end = 128, predicted length 12.
SCRIPT_A = {
    # step 0: masked slots 4..7; two confidences reach 0.9 -> slots 5, 7 accepted
    0: {"rows": {4: (1, 0.5), 5: (2, 0.95), 6: (3, 0.3), 7: (4, 0.92)},
        "scores": {0: 0.3, 1: 0.1, 2: 0.3, 3: 0.2}},
    # step 1: masked 4, 6, 8, 9; none reaches 0.9 -> only the best (slot 6) accepted
    1: {"rows": {4: (5, 0.2), 6: (5, 0.6), 8: (6, 0.4), 9: (7, 0.1)},
        "scores": {1: 0.5, 3: 0.4, 2: 0.0, 0: 0.9, 5: 0.2, 7: 0.2}},
    # step 2: masked 8, 4, 9, 10; EOS accepted at slot 8 -> predicted length 9
    2: {"rows": {8: (EOS, 0.95), 4: (1, 0.5), 9: (2, 0.3), 10: (3, 0.2)}},
    # step 3: masked 4, 9, 10, 11; slots 9.. are past the predicted length: their
    # confidences are zeroed (slot 10's 0.95 must not win), so slot 4 is accepted
    3: {"rows": {4: (1, 0.3), 9: (2, 0.5), 10: (3, 0.95), 11: (4, 0.2)}},
}


@pytest.mark.parametrize("impl", IMPLS)
def test_pass1_acceptance_ranking_and_eos_length_mask(impl):
    model = Scripted(SCRIPT_A)
    resp, nt, mx, n_steps = _run(impl, model, [P0], 1, **_kw())
    c = model.calls
    assert [r["step"] for r in c] == [0, 1, 2, 3]
    # step 0: the masked block, then every other key slot as tracked rows
    assert c[0]["qpos"] == [4, 5, 6, 7] + [0, 1, 2, 3] + list(range(8, 128))
    assert c[0]["masked_blocks"] == [[0, 128, 0, 4]]
    assert c[0]["tracked_blocks"] == [[0, 128, 4 + 4 * i, min(8 + 4 * i, 128)] for i in range(31)]
    # after step 0: slots 5, 7 decoded (conf order 5, 7 | 4, 6); full_pos[:4] = 0..3 sorted
    # by score (1: 0.1, 3: 0.2, then 0.3 at slots 0 and 2 -> higher slot first: 2, 0)
    # -> full_pos = [1, 3, 2, 0, 5, 7, 4, 6, 8, ...], nd = 6
    assert c[1]["qpos"] == [4, 6, 8, 9] + [2, 0, 5, 7]
    assert c[1]["x"] == [MASK] * 4 + [P0[2], P0[0], 2, 4]
    assert c[1]["masked_blocks"] == [[0, 128, 0, 4]]
    assert c[1]["tracked_blocks"] == [[0, 128, 4, 8]]
    # after step 1: slot 6 decoded (token 5); conf order 6, 8, 4, 9; scores rank
    # [1, 3, 2, 0, 5, 7] as 2 (0.0), 7, 5 (0.2 tie: higher first), 3, 1, 0
    # -> full_pos = [2, 7, 5, 3, 1, 0, 6, 8, 4, 9, 10, ...], nd = 7
    assert c[2]["qpos"] == [8, 4, 9, 10] + [3, 1, 0, 6]
    # after step 2: EOS at slot 8; scores all zero -> [7, 6, 5, 3, 2, 1, 0]; nd = 8
    assert c[3]["qpos"] == [4, 9, 10, 11] + [2, 1, 0, 8]
    # step 3 accepts slot 4 (token 1); every position below 9 is decoded: done
    assert resp[0] == [1, 2, 5, 4, EOS]
    assert (nt, mx, n_steps) == (5, 8, [4])


@pytest.mark.parametrize("impl", IMPLS)
def test_pass1_nan_confidence_ranks_first(impl):
    """x0_p.sort(descending=True) (generate.py:343) puts NaN first, as torch sorts it: with
    no confidence at the threshold, keep = 1 takes the NaN row (slot 5), whose token is
    torch.max's index for an all-NaN softmax row (0), and not the best number (slot 4)."""
    script = {0: {"rows": {4: (1, 0.5), 5: (2, float("nan")), 6: (3, 0.3), 7: (4, 0.2)}}}
    model = Scripted(script)
    resp, _, _, _ = _run(impl, model, [P0], 1, **_kw())
    c = model.calls
    # after step 0: full_pos[4:8] = [5, 4, 6, 7], nd = 5; full_pos[:4] = 0..3 all at score 0
    # -> higher slot first: [3, 2, 1, 0]; tracked = full_pos[1:5] = [2, 1, 0, 5]
    assert c[1]["qpos"] == [4, 6, 7, 8] + [2, 1, 0, 5]
    assert c[1]["x"] == [MASK] * 4 + [P0[2], P0[1], P0[0], 0]
    assert resp[0][:2] == [3, 0]  # slot 4 by the default row at step 1, slot 5 the NaN row's


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("track,mask_num,tracked", [
    (1, 1, [2, 0, 5, 7]),                                   # last bm decoded entries
    (2, 1, [1, 3, 2, 0, 5, 7]),                             # 2 bm entries, clipped at 0
    (1, 2, [2, 0, 5, 7, 10, 11, 12, 13]),                   # + look-ahead full_pos[10:14]
    (-1, 1, [1, 3, 2, 0, 5, 7] + list(range(10, 128))),     # every other slot
])
def test_tracked_set(impl, track, mask_num, tracked):
    model = Scripted(SCRIPT_A)
    _run(impl, model, [P0], 1, **_kw(track_num=track, mask_num=mask_num))
    # after step 0: full_pos = [1, 3, 2, 0, 5, 7, 4, 6, 8, 9, 10, ...], nd = 6
    assert model.calls[1]["qpos"] == [4, 6, 8, 9] + tracked


# Prompt of 8 tokens, gen 8, block 4, verify: L = 128, k_end = 128, predicted length 16.
P1 = [1, 2, 3, 4, 5, 6, 7, 8]
SCRIPT_B = {
    0: {"rows": {8: (1, 0.3), 9: (2, 0.95), 10: (3, 0.6), 11: (4, 0.4)},
        "scores": {3: 0.5, 9: 0.7, 0: -0.1},
        # mask-view rows of the candidates (rows T + S .. T + 2S - 1 = 6, 7): the draft
        # tokens 3 and 4 at probabilities 0.95 and 0.92 -> cumprod 0.95, 0.874 -> keep 1
        "verify_rows": {6: (3, 0.95), 7: (4, 0.92)}},
}


@pytest.mark.parametrize("impl", IMPLS)
def test_verify_lists_mask_and_cumprod_acceptance(impl):
    model = Scripted(SCRIPT_B)
    resp, nt, mx, n_steps = _run(impl, model, [P1], 1, **_kw(verify=True))
    c = model.calls
    assert [(r["step"], r["verify"]) for r in c[:3]] == [(0, False), (0, True), (1, False)]
    # pass 1: conf order 9, 10, 11, 8 -> full_pos[8:12] = [9, 10, 11, 8]; keep 1 (slot 9,
    # token 2), nd = 9; S = min(4 - 1, 2) = 2 candidates [10, 11]; T = 8 - 4 = 4 fill rows
    # full_pos[5:9] = [5, 6, 7, 9]
    v = c[1]
    assert v["qpos"] == [5, 6, 7, 9, 10, 11, 10, 11]
    # rows: fill tokens, drafts of the candidates (tokens 3, 4), the candidates' [MASK]s
    assert v["x"] == [6, 7, 8, 2, 3, 4, MASK, MASK]
    # keys: full_pos[:nd - T] = 0..4 and full_pos[nd + S : 128] = [8, 12, 13, ..., 127]
    assert v["keys"] == [0, 1, 2, 3, 4, 8] + list(range(12, 128))
    assert v["vblocks"] == [[0, 122, 0, 8]]
    exp_mask = np.ones((8, 8), bool)
    exp_mask[:4, 4:6] = False                      # fill rows do not see the drafts
    exp_mask[4:8, 4:8] = [[1, 0, 0, 1],            # draft 0: draft 0, mask 1
                          [1, 1, 0, 0],            # draft 1: drafts 0-1, no mask
                          [0, 0, 1, 1],            # mask 0: masks 0-1
                          [1, 0, 0, 1]]            # mask 1: draft 0, mask 1
    np.testing.assert_array_equal(v["mask"], exp_mask)
    # verify accepts 1 (slot 10, token 3): nd = 10; the ranked segment is full_pos[:10 - 1]
    # = [0, .., 7, 9]: 0 (-0.1), zeros 7, 6, 5, 4, 2, 1, then 3 (0.5), 9 (0.7)
    # -> full_pos = [0, 7, 6, 5, 4, 2, 1, 3, 9, 10, 11, 8, 12, ...]
    assert c[2]["qpos"] == [11, 8, 12, 13] + [1, 3, 9, 10]
    # step 1: masked [11, 8, 12, 13] at the default confidence 0.95: all four accepted in
    # pass 1 (nd = 14), so S = 0 and the verify forward holds T = 8 fill rows
    # full_pos[6:14] = [1, 3, 9, 10, 11, 8, 12, 13] and accepts nothing; all scores are 0, so
    # full_pos[:14] becomes the slots in descending order, and the next masked block is
    # full_pos[14:18] = [14, 15, 16, 17] (positions past prompt + gen are decoded too)
    passes = [r for r in c if not r["verify"]]
    verifies = [r for r in c if r["verify"]]
    assert passes[2]["qpos"] == [14, 15, 16, 17] + [3, 2, 1, 0]
    # step 2 accepts all four (nd = 18); nothing below the predicted length 16 is left
    assert len(passes) == 3
    if impl == "oracle":
        # the reference runs the candidate-free verify forwards of steps 1 and 2 too
        assert len(verifies) == 3
        v1 = verifies[1]
        assert v1["step"] == 1 and v1["qpos"] == [1, 3, 9, 10, 11, 8, 12, 13]
        assert v1["keys"] == [0, 7, 6, 5, 4, 2] + list(range(14, 128))
        assert v1["mask"].all()
    else:
        # the product skips a verify forward without candidate rows: it reads no logits and
        # writes no cache rows or scores, so every decision is the same
        assert len(verifies) == 1
    # response = slots 8..17: 8 -> 3 (step 1), 9 -> 2 (pass 1), 10 -> 3 (verify), the rest 3
    assert resp[0] == [3, 2, 3, 3, 3, 3, 3, 3, 3, 3]
    assert (nt, mx, n_steps) == (10, 8, [3])


# Two prompts through one row: refill after the first finishes.
P2 = [7, 8, 9, 10, 11, 12]


@pytest.mark.parametrize("impl", IMPLS)
def test_refill_loads_next_prompt(impl):
    # step 0 accepts all four masked slots of prompt 0 (gen 4: predicted length 8) -> done
    script = {0: {"rows": {4: (1, 0.95), 5: (2, 0.95), 6: (3, 0.95), 7: (4, 0.95)}},
              1: {"rows": {6: (5, 0.95), 7: (6, 0.95), 8: (7, 0.95), 9: (8, 0.95)}}}
    model = Scripted(script)
    resp, nt, mx, n_steps = _run(impl, model, [P0, P2], 1, **_kw(gen_length=4))
    c = model.calls
    assert len(c) == 2
    # stride L = ((6 + 4 + 4) // 128 + 1) * 128 = 128; prompt 1 (6 tokens) starts over:
    # masked 6..9, tracked 0..5 and 10..127 (k_end 128), x = prompt, masks, EOS from 10
    assert c[1]["qpos"] == [6, 7, 8, 9] + [0, 1, 2, 3, 4, 5] + list(range(10, 128))
    assert c[1]["x"] == [MASK] * 4 + P2 + [EOS] * 118
    assert c[1]["masked_blocks"] == [[0, 128, 0, 4]]
    assert resp == [[1, 2, 3, 4], [5, 6, 7, 8]]
    assert (nt, mx, n_steps) == (8, 8, [1, 1])
