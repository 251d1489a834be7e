"""Greedy decoding of a trained model through the HIP path, compared position by position
with a float32 copy of the same model.

Random weights give near-tied logits, where any bf16 arithmetic flips argmaxes; a trained
model's decisions are not near ties. fdl.copy_task trains a small LLaDA-shaped model (2
layers, d_model 256, two heads of 128) with the masked-diffusion objective on a copy task
(prompt of 32 tokens, response = the prompt twice, then EOS) in float32 on the GPU; fresh
prompts are then decoded with the reference's Flash-Cache (+ Flash-Verify) loop
(generate_with_Flash_dLLM, block 32, gamma 0.9) twice: the bf16 model on the HIP kernels and
the float32 model on the unfused torch driver. Every decoded position must agree (the
reference's greedy-decoding criterion asks for 99% of positions), and the decode must be
right on the task."""
import numpy as np
import pytest
import torch

from flash_cache_hip import flash_fused_elastic_cache
from fdl.copy_task import (CONFIG, GEN_LEN, N_TOKENS, PROMPT_LEN, compare_decodes,
                           train_copy_model)
from fdl.generate import DecodeStats, generate_with_Flash_dLLM
from fdl.model import LLaDAConfig, build_model
from fdl.torch_path import flash_fused_elastic_cache_torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def models():
    twin, acc, gap = train_copy_model(DEV, flash_fused_elastic_cache_torch)
    print(f"trained: masked-token accuracy {acc:.4f}, smallest top-2 logit gap {gap:.2f}")
    assert acc >= 0.999 and gap > 1.0
    hip = build_model(LLaDAConfig(**CONFIG), flash_fused_elastic_cache, DEV, torch.bfloat16)
    hip.load_state_dict({k: v.to(torch.bfloat16) for k, v in twin.state_dict().items()})
    return hip, twin


# threshold 0.9: the trained model passes it with every masked token, so a block decodes in
# one step; 1.01: pass 1 keeps one token per step (keep = max(#conf >= threshold, 1)), so
# the decode runs a step per token with tracked refreshes, and Flash-Verify accepts drafts
# (verify, device_schedule, threshold, kv_pages, block_length, track_num, mask_num)
CASES = [
    (False, False, 0.9, None, 32, 1, 1), (False, False, 1.01, None, 32, 1, 1),
    (True, False, 1.01, None, 32, 1, 1), (True, True, 1.01, None, 32, 1, 1),
    (True, True, 1.01, 12, 32, 1, 1),
    # other block lengths (verify needs a prompt of 2 blocks: not at block 64), and more
    # tracked / look-ahead blocks
    (True, True, 1.01, None, 16, 1, 1), (False, False, 1.01, None, 64, 1, 1),
    (False, True, 1.01, None, 16, 2, 2), (True, True, 1.01, None, 16, -1, 2),
]


@pytest.mark.parametrize("verify,device_schedule,threshold,kv_pages,block,track,mask", CASES)
def test_trained_model_greedy_decode_matches_float32(models, verify, device_schedule, threshold,
                                                     kv_pages, block, track, mask):
    """Twelve fresh prompts, three batch rows (refills); every decoded position of the HIP
    bf16 decode equals the float32 decode's, and both copy the prompt."""
    hip, twin = models
    rng = np.random.default_rng(11)
    n = 12
    prompts = [torch.from_numpy(rng.integers(0, N_TOKENS, PROMPT_LEN)) for _ in range(n)]
    kw = dict(gen_length=GEN_LEN, block_length=block, mask_id=63, eos_id=62,
              threshold=threshold, gamma=0.9, track_num=track, mask_num=mask, verify=verify)
    st_h, st_t = DecodeStats(), DecodeStats()
    r_h, _, _ = generate_with_Flash_dLLM(hip, prompts, [PROMPT_LEN] * n, 3, [None] * n, [0] * n,
                                         stats=st_h, device_schedule=device_schedule,
                                         kv_pages=kv_pages, **kw)
    r_t, _, _ = generate_with_Flash_dLLM(twin, prompts, [PROMPT_LEN] * n, 3, [None] * n,
                                         [0] * n, stats=st_t, use_gpu_rank=False, **kw)
    c = compare_decodes(prompts, r_h, r_t)
    print(f"verify={verify} device_schedule={device_schedule} threshold={threshold} "
          f"kv_pages={kv_pages} block={block} track={track} mask={mask}: {c}; steps "
          f"{st_h.steps} (float32 {st_t.steps}), verify accepted {st_h.verify_accepted}")
    assert c["content_mismatch"] == 0
    assert c["positions"] >= n * GEN_LEN
    assert c["agreement"] >= 0.99
    assert c["right"] >= 0.99
    if verify:
        assert st_h.verify_accepted > 0  # drafts of a confident model pass gamma


@pytest.mark.parametrize("verify", [False, True])
def test_trained_model_reference_loop_through_hip_driver(models, verify):
    """The reference's decode loop, restated statement for statement
    (oracle/generate_oracle.py; info = [], int64 block tables, the dense verify mask), driving
    the HIP drop-in driver on the trained model: the same tokens, token counts and
    per-prompt step counts as the product loop (fdl.generate) on the same kernels, with
    refills (six prompts, three rows) and, with Flash-Verify, accepted drafts; and the task's
    answer."""
    from oracle.generate_oracle import generate_oracle
    hip, _ = models
    rng = np.random.default_rng(3)
    n = 6
    prompts = [torch.from_numpy(rng.integers(0, N_TOKENS, PROMPT_LEN)) for _ in range(n)]
    kw = dict(gen_length=GEN_LEN, block_length=32, mask_id=63, threshold=1.01, gamma=0.9,
              track_num=1, mask_num=1, verify=verify)
    steps_o = [0] * n
    resp_o, nt_o, mx_o = generate_oracle(hip, prompts, [PROMPT_LEN] * n, 3, steps_o, eos_id=62,
                                         **kw)
    steps_p = [0] * n
    st = DecodeStats()
    resp_p, nt_p, mx_p = generate_with_Flash_dLLM(hip, prompts, [PROMPT_LEN] * n, 3, [None] * n,
                                                  steps_p, eos_id=62, use_gpu_rank=False,
                                                  stats=st, **kw)
    print(f"verify={verify}: steps {steps_o} / {steps_p}, tokens {nt_o} / {nt_p}, verify "
          f"accepted {st.verify_accepted}")
    assert steps_p == steps_o and (nt_p, mx_p) == (nt_o, mx_o)
    for i in range(n):
        assert resp_p[i] == resp_o[i], i
    c = compare_decodes(prompts, resp_p, resp_o)
    assert c["right"] >= 0.99
    if verify:
        assert st.verify_accepted > 0
