"""The hot-path chain captured in a HIP graph and replayed several times.

bench.py measures the single-layer chain from graph replays, and a decode loop may capture
its steps. Each replay here follows eager work of the program's own (the chain's state
reset, the outputs poisoned, an unrelated product) and a synchronisation, and every replay
must equal the eagerly launched chain bit for bit. The chain: fused QKV + RoPE + cache
write, block attention with softmax-colsum importance (workspace), the last layer's head
reduction folded into the top-k ranking (which permutes the decoded-slot lists in place),
and block attention with raw importance on a grid small enough for the key split (partial
rows in a workspace that fdl.ops allocates during capture, then the merge kernel)."""
import numpy as np
import pytest
import torch

from fdl import lib, ops
from fdl.generate import get_rotary_embedding
from fdl.schedule import contiguous_page_table, make_plan, seqs_from_reference_blocks

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
B, L, K_END, BM, TRACK, H, TOPK = 4, 512, 384, 32, 16, 8, 16
D = 128 * H


def _inputs(seed: int) -> dict:
    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    frontier = 128 + 32 * rng.integers(0, 6, B)
    masked = [b * L + np.arange(f, f + BM) for b, f in enumerate(frontier)]
    tracked = [b * L + rng.choice(int(f), TRACK, replace=False) for b, f in enumerate(frontier)]
    slots = np.concatenate(masked + tracked).astype(np.int64)
    mb = np.array([[b, K_END, BM * b, BM * (b + 1)] for b in range(B)])
    tb = np.array([[b, K_END, B * BM + TRACK * b, B * BM + TRACK * (b + 1)] for b in range(B)])
    sin_l, cos_l = get_rotary_embedding(L, 128, 500000.0, "cpu")
    d = dict(
        x=torch.randn((len(slots), D), generator=gen).to(torch.bfloat16),
        w=[(torch.randn((D, D), generator=gen) * 0.02).to(torch.bfloat16) for _ in range(3)],
        kc=torch.randn((B * L, D), generator=gen).to(torch.bfloat16),
        vc=torch.randn((B * L, D), generator=gen).to(torch.bfloat16),
        sin=sin_l.repeat(B, 1), cos=cos_l.repeat(B, 1), slot=torch.from_numpy(slots),
        full_pos=torch.arange(B * L, dtype=torch.int64).reshape(B, L),
        seg=torch.tensor([[b * L, int(f)] for b, f in enumerate(frontier)], dtype=torch.int32),
        seg_keys=torch.tensor([[b, K_END] for b in range(B)], dtype=torch.int32))
    d = {k: [t.to(DEV) for t in v] if isinstance(v, list) else v.to(DEV) for k, v in d.items()}
    d["plan"] = make_plan(seqs_from_reference_blocks(mb, tb, importance=True),
                          contiguous_page_table(B, L), device=DEV)
    d["max_len"] = int(frontier.max())
    return d


def test_hot_path_chain_graph_replays_equal_eager():
    d = _inputs(5)
    Q = d["x"].shape[0]
    scale = 1.0 / np.sqrt(128)
    plan = d["plan"]
    assert plan.n_work * H * 4 <= 256  # the raw-importance launch takes the key split
    kc0, vc0, pos0 = d["kc"].clone(), d["vc"].clone(), d["full_pos"].clone()
    kc, vc, full_pos = d["kc"], d["vc"], d["full_pos"]
    q = torch.empty((Q, D), dtype=torch.bfloat16, device=DEV)
    att = torch.empty_like(q)
    att2 = torch.empty_like(q)
    imp = torch.empty((H, B * L), dtype=torch.float32, device=DEV)
    imp2 = torch.empty_like(imp)
    scores = torch.empty(B * L, dtype=torch.float32, device=DEV)
    topk = torch.empty((B, TOPK), dtype=torch.int64, device=DEV)
    ws = torch.empty(max(ops.attention_workspace_floats(plan, H), 4), dtype=torch.float32,
                     device=DEV)
    outs = (q, att, att2, imp, imp2, scores, topk, full_pos)

    def reset():
        # the chain's state as the step starts; outputs poisoned
        kc.copy_(kc0)
        vc.copy_(vc0)
        full_pos.copy_(pos0)
        scores.zero_()
        imp.zero_()
        imp2.zero_()
        for t in (q, att, att2):
            t.fill_(float("nan"))
        topk.fill_(-7)

    def chain():
        ops.qkv_rope_cache(d["x"], *d["w"], d["sin"], d["cos"], d["slot"], q, kc, vc, H)
        ops.block_attention(q, kc, vc, plan, att, H, scale, lib.IMP_SOFTMAX_COLSUM, imp,
                            workspace=ws)
        ops.importance_rank(scores, full_pos, d["seg"], d["max_len"], topk, TOPK, imp_part=imp,
                            scale=1.0, plan=plan, seg_keys=d["seg_keys"])
        ops.block_attention(q, kc, vc, plan, att2, H, scale, lib.IMP_RAW_LOGIT, imp2)

    reset()
    chain()
    torch.cuda.synchronize()
    eager = [t.clone() for t in outs] + [kc[d["slot"]].clone(), vc[d["slot"]].clone()]
    assert not torch.isnan(att.float()).any() and not torch.isnan(att2.float()).any()
    assert (topk >= 0).all()

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        reset()
        chain()  # warm call on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        chain()
    torch.cuda.synchronize()

    other = torch.randn((512, 512), device=DEV)
    for rep in range(4):
        reset()
        other = torch.tanh(other @ other.T / 512)  # unrelated eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in outs] + [kc[d["slot"]].clone(), vc[d["slot"]].clone()]
        names = ("q", "att", "att2", "imp", "imp2", "scores", "topk", "full_pos", "k rows",
                 "v rows")
        for n, a, e in zip(names, got, eager):
            assert torch.equal(a, e), f"replay {rep}: {n} differs from the eager chain"


def test_flash_verify_pair_graph_replays_equal_eager():
    """The Flash-Verify pair in one graph: the packed projection of the draft / mask rows
    (K and V to packed rows, the cache untouched) and the verify attention with the
    closed-form (T, S) masks over each block's key list, on a grid of 40 blocks x 8 heads
    (more than one round: two heads per workgroup)."""
    Hv, n_blk, Lv, bm = 8, 40, 512, 32
    rows, Dv = 2 * bm, 128 * 8
    rng = np.random.default_rng(17)
    gen = torch.Generator().manual_seed(17)
    key_pos, vblocks, ts, qslots = [], [], [], []
    acc = 0
    for j in range(n_blk):
        S = int(rng.integers(1, bm + 1))
        T = rows - 2 * S
        nd = int(rng.integers(T + 64, Lv - S - 1))
        fill, cand = np.arange(nd - T, nd), np.arange(nd, nd + S)
        keys = np.concatenate([np.arange(nd - T), np.arange(nd + S, Lv)]) + j * Lv
        key_pos.append(keys)
        vblocks.append((acc, acc + len(keys), j * rows, (j + 1) * rows))
        acc += len(keys)
        ts.append((T, S))
        qslots.append(np.concatenate([fill, cand, cand]) + j * Lv)
    Q = n_blk * rows
    sin_l, cos_l = get_rotary_embedding(Lv, 128, 500000.0, "cpu")
    x = torch.randn((Q, Dv), generator=gen).to(torch.bfloat16).to(DEV)
    w = [(torch.randn((Dv, Dv), generator=gen) * 0.02).to(torch.bfloat16).to(DEV)
         for _ in range(3)]
    kc = torch.randn((n_blk * Lv, Dv), generator=gen).to(torch.bfloat16).to(DEV)
    vc = torch.randn((n_blk * Lv, Dv), generator=gen).to(torch.bfloat16).to(DEV)
    sin, cos = sin_l.repeat(n_blk, 1).to(DEV), cos_l.repeat(n_blk, 1).to(DEV)
    slot = torch.from_numpy(np.concatenate(qslots).astype(np.int64)).to(DEV)
    kp = torch.from_numpy(np.concatenate(key_pos).astype(np.int64)).to(DEV)
    vb = torch.tensor(vblocks, dtype=torch.int32, device=DEV)
    tsd = torch.tensor(ts, dtype=torch.int32, device=DEV)
    assert n_blk * Hv > 256
    q, k1, v1, out = (torch.empty((Q, Dv), dtype=torch.bfloat16, device=DEV) for _ in range(4))
    kc0 = kc.clone()
    scale = 1.0 / np.sqrt(128)

    def reset():
        for t in (q, k1, v1, out):
            t.fill_(float("nan"))

    def pair():
        ops.qkv_rope_cache(x, *w, sin, cos, slot, q, k1, v1, Hv, kv_packed=True)
        ops.verify_attention(q, k1, v1, kc, vc, kp, vb, tsd, rows, out, Hv, scale)

    reset()
    pair()
    torch.cuda.synchronize()
    eager = [t.clone() for t in (q, k1, v1, out)]
    assert not torch.isnan(out.float()).any()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pair()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        pair()
    torch.cuda.synchronize()
    other = torch.randn((512, 512), device=DEV)
    for rep in range(4):
        reset()
        other = torch.tanh(other @ other.T / 512)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for n, a, e in zip(("q", "k1", "v1", "out"), (q, k1, v1, out), eager):
            assert torch.equal(a, e), f"replay {rep}: {n} differs from the eager pair"
    assert torch.equal(kc, kc0)  # the packed projection leaves the cache untouched
