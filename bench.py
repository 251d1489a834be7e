#!/usr/bin/env python3
"""Benchmark of the Flash-Cache hot path on one MI355X.

One step = one transformer layer's hot path on the bf16 single-layer workload:
batch 8, KV cache of 768 keys per sequence (slot stride 896), denoising block 32; the
query is each sequence's 32-row masked block plus 32 tracked rows (random unique decoded
slots), 512 rows in all; d_model 4096, 32 heads x 128, RoPE theta 5e5.
    1. fused QKV projection + RoPE + K/V cache write       (fdl_qkv_rope_cache)
    2. block-table attention, masked and tracked rows of a sequence in one tile, with
       attention-importance = column sums of softmax(QK^T/sqrt(128)) over the masked
       rows                                                  (fdl_block_attention)
    3. the step's ranking, as at a step's last layer: the layer's head reduction of the
       importance into the scores of every key, then the top-32 of the decoded slots, in
       one launch                                            (fdl_importance_accumulate_rank)
       (at the other layers, step 3 is the head reduction alone, fdl_importance_accumulate)

    python bench.py [--steps K] [--warmup W] [--no-cpu]

Prints one JSON line (value = microseconds per layer, lower is better). Per-kernel times
come from HIP events recorded on the stream the kernels run on, around every launch in the
timed region. The CPU baseline times the numpy oracle (the reference algorithm restated on
the CPU) on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT / "flash-dllm_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "µs/layer fused cache-update+attn (HBM GB/s, MFMA %); LLaDA-8B tokens/s"
PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0

D, H, HD = 4096, 32, 128
B, L, K_END, BM, TRACK, TOPK = 8, 896, 768, 32, 32, 32
THETA = 500000.0


def build_workload(seed: int, device):
    """Seeded synthetic inputs of the single-layer bf16 workload (host and device)."""
    import torch
    from fdl.schedule import contiguous_page_table, make_plan, seqs_from_reference_blocks

    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    frontier = 256 + 32 * rng.integers(0, 16, B)
    masked = [b * L + np.arange(f, f + BM) for b, f in enumerate(frontier)]
    tracked = [b * L + rng.choice(int(f), TRACK, replace=False) for b, f in enumerate(frontier)]
    slots = np.concatenate(masked + tracked).astype(np.int64)
    Q = len(slots)
    # reference block tables (batch, k_end, q0, q1): masked blocks, then tracked blocks
    mb = np.array([[b, K_END, BM * b, BM * (b + 1)] for b in range(B)])
    tb = np.array([[b, K_END, B * BM + TRACK * b, B * BM + TRACK * (b + 1)] for b in range(B)])
    w = {
        "x": (torch.randn((Q, D), generator=gen)).to(torch.bfloat16),
        "wq": (torch.randn((D, D), generator=gen) * 0.02).to(torch.bfloat16),
        "wk": (torch.randn((D, D), generator=gen) * 0.02).to(torch.bfloat16),
        "wv": (torch.randn((D, D), generator=gen) * 0.02).to(torch.bfloat16),
        "x_prefill": (torch.randn((B * K_END, D), generator=gen)).to(torch.bfloat16),
    }
    inv = 1.0 / (THETA ** (np.arange(0, HD, 2, dtype=np.float32) / np.float32(HD)))
    ang = np.outer(np.arange(L, dtype=np.float32), inv.astype(np.float32)).astype(np.float32)
    ang = np.concatenate([ang, ang], axis=1)
    sin = np.tile(np.sin(ang).astype(np.float32), (B, 1))
    cos = np.tile(np.cos(ang).astype(np.float32), (B, 1))
    host = dict(slots=slots, mb=mb, tb=tb, frontier=frontier, sin=sin, cos=cos, **w)
    dev = None
    if device is not None:
        dev = {k: v.to(device) for k, v in w.items()}
        dev["sin"] = torch.from_numpy(sin).to(device)
        dev["cos"] = torch.from_numpy(cos).to(device)
        dev["slot"] = torch.from_numpy(slots).to(device)
        dev["plan"] = make_plan(seqs_from_reference_blocks(mb, tb, importance=True),
                                contiguous_page_table(B, L), device=device)
        dev["plan"].validate(Q, B * L)
        full_pos = np.arange(B * L, dtype=np.int64).reshape(B, L)
        dev["full_pos"] = torch.from_numpy(full_pos).to(device)
        dev["seg_keys"] = torch.from_numpy(np.array([[b, K_END] for b in range(B)],
                                                    dtype=np.int32)).to(device)
        dev["seg"] = torch.from_numpy(np.array([[b * L, int(f)] for b, f in enumerate(frontier)],
                                               dtype=np.int32)).to(device)
    return host, dev


def algorithmic_counts(Q: int) -> dict:
    """Per-launch algorithmic flops / bytes (each byte counted once)."""
    qkv_f = 2.0 * Q * D * 3 * D
    qkv_b = 3.0 * D * D * 2 + Q * D * 2 + Q * D * 2 + 2.0 * Q * D * 2 + Q * HD * 4 * 2 + Q * 8
    rows = (BM + TRACK)
    attn_f = B * 4.0 * rows * K_END * D + B * 2.0 * BM * K_END * D  # + importance pass
    attn_b = B * (2.0 * rows * D * 2 + 2.0 * K_END * D * 2) + B * K_END * H * 4
    return dict(qkv=(qkv_f, qkv_b), attn=(attn_f, attn_b))


TRAFFIC_FILE = ROOT / "profiles" / "single_layer_bf16_hbm_traffic.txt"


def measured_traffic() -> dict:
    """HBM bytes per launch of each kernel, from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (counters scaled by a 100 MiB copy; see the file's header)."""
    out = {}
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic":
                out[parts[1]] = int(parts[2])
    except OSError:
        pass
    return out


def run_gpu(steps: int, warmup: int, seed: int = 2):
    import torch
    from fdl import lib, ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    host, d = build_workload(seed, dev)
    Q = len(host["slots"])
    kc = torch.zeros((B * L, D), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    # prefill: every key slot of every sequence gets a K/V from the same fused kernel
    pre_slots = torch.from_numpy(
        np.concatenate([b * L + np.arange(K_END) for b in range(B)]).astype(np.int64)).to(dev)
    qtmp = torch.empty((B * K_END, D), dtype=torch.bfloat16, device=dev)
    ops.qkv_rope_cache(d["x_prefill"], d["wq"], d["wk"], d["wv"], d["sin"], d["cos"], pre_slots,
                       qtmp, kc, vc, H)
    del qtmp
    q = torch.empty((Q, D), dtype=torch.bfloat16, device=dev)
    att = torch.empty_like(q)
    imp = torch.zeros((H, B * L), dtype=torch.float32, device=dev)
    scores = torch.zeros(B * L, dtype=torch.float32, device=dev)
    topk = torch.empty((B, TOPK), dtype=torch.int64, device=dev)
    plan = d["plan"]
    scale = 1.0 / np.sqrt(HD)
    max_len = int(host["frontier"].max())
    names = ["qkv_rope_cache", "block_attention", "importance_accumulate_rank"]

    def step(ev=None):
        def mark(i):
            if ev is not None:
                ev[i].record()
        mark(0)
        ops.qkv_rope_cache(d["x"], d["wq"], d["wk"], d["wv"], d["sin"], d["cos"], d["slot"], q,
                           kc, vc, H)
        mark(1)
        ops.block_attention(q, kc, vc, plan, att, H, scale, lib.IMP_SOFTMAX_COLSUM, imp)
        mark(2)
        # the step's last layer: its head reduction folded into the top-32 ranking
        ops.importance_rank(scores, d["full_pos"], d["seg"], max_len, topk, TOPK, imp_part=imp,
                            scale=1.0, plan=plan, seg_keys=d["seg_keys"])
        mark(3)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # pass 1: whole-step time, no events between kernels
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        step()
    t1.record()
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    # pass 2: per-kernel durations from events around every launch
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
           for _ in range(steps)]
    for i in range(steps):
        step(evs[i])
    torch.cuda.synchronize()
    per = {n: float(np.mean([evs[i][k].elapsed_time(evs[i][k + 1]) for i in range(steps)]) * 1e3)
           for k, n in enumerate(names)}
    return dict(Q=Q, total_ms=total_ms, per_kernel_us=per)


def run_torch_layer(reps: int = 20, seed: int = 2) -> dict:
    """The same single-layer chain with unfused PyTorch ops on the same GPU (the
    conventional path the reference's fused kernels are compared with), batched over the
    sequences (all 8 have 64 query rows and 768 keys): F.linear Q/K/V, rotate-half RoPE on
    gathered sin/cos rows, index_copy_ into the caches, K/V head slices gathered from the
    caches, one batched QK^T and one PV product (bf16, contiguous operands; float32
    softmax), softmax column sums of the masked rows into the scores, then a sort of each
    sequence's decoded slots and its top-32."""
    import torch
    import torch.nn.functional as F
    from fdl.torch_path import _rotate

    dev = torch.device("cuda:0")
    host, d = build_workload(seed, dev)
    bf = torch.bfloat16
    slots = d["slot"]
    kc = torch.zeros((B * L, D), dtype=bf, device=dev)
    vc = torch.zeros_like(kc)
    pre = torch.from_numpy(np.concatenate([b * L + np.arange(K_END) for b in range(B)])).to(dev)
    sp, cp = d["sin"][pre], d["cos"][pre]
    kc.index_copy_(0, pre, _rotate(F.linear(d["x_prefill"], d["wk"]), sp, cp, H).to(bf))
    vc.index_copy_(0, pre, F.linear(d["x_prefill"], d["wv"]))
    sin_r, cos_r = d["sin"][slots], d["cos"][slots]
    scale = 1.0 / np.sqrt(HD)
    mb, tb = host["mb"], host["tb"]
    rows = torch.from_numpy(np.stack([np.concatenate([np.arange(mb[b][2], mb[b][3]),
                                                      np.arange(tb[b][2], tb[b][3])])
                                      for b in range(B)])).to(dev)          # [B, 64]
    nr = rows.shape[1]
    decoded = [torch.arange(b * L, b * L + int(f), device=dev) for b, f in enumerate(host["frontier"])]

    def step():
        x = d["x"]
        q = _rotate(F.linear(x, d["wq"]), sin_r, cos_r, H).to(bf)
        k = _rotate(F.linear(x, d["wk"]), sin_r, cos_r, H).to(bf)
        v = F.linear(x, d["wv"])
        kc.index_copy_(0, slots, k)
        vc.index_copy_(0, slots, v)
        kt = kc.view(B, L, H, HD)[:, :K_END].permute(0, 2, 3, 1).contiguous()  # [B, H, hd, K]
        vh = vc.view(B, L, H, HD)[:, :K_END].permute(0, 2, 1, 3).contiguous()  # [B, H, K, hd]
        qh = q[rows].view(B, nr, H, HD).permute(0, 2, 1, 3).contiguous()       # [B, H, 64, hd]
        p = torch.softmax(torch.matmul(qh, kt).float() * scale, dim=-1)
        o = torch.matmul(p.to(bf), vh)
        att = torch.empty_like(q)
        att[rows.reshape(-1)] = o.permute(0, 2, 1, 3).reshape(B * nr, D)
        colsum = p[:, :, :BM].sum(dim=(1, 2))                                  # [B, K]
        scores = torch.zeros(B, L, dtype=torch.float32, device=dev)
        scores[:, :K_END] += colsum
        scores = scores.view(-1)
        for b in range(B):
            order = torch.sort(scores[decoded[b]]).indices
            decoded[b][order[-TOPK:]]
        return att

    us = _time_op(step, reps)
    return {"us": round(us, 2), "what": "the same layer chain with unfused PyTorch ops batched "
            "over the sequences (conventional path), same GPU, events over " + str(reps) + " steps"}


def _time_op(fn, reps: int, warm: int = 3) -> float:
    """Mean microseconds per call of fn() on the current stream (events around the loop)."""
    import torch
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def run_configs(seed: int = 3, reps: int = 10) -> dict:
    """Secondary measurements on the other single-layer workloads (bf16, d_model 4096, 32
    heads): the block-table stress batch (32 sequences, caches of 512-1536 keys in randomly
    permuted 32-slot pages, a quarter of them full recomputes), its full-recompute tiles on
    their own, and the Flash-Verify batch (16 sequences, 1024-slot caches, 4-32 candidates
    each as draft and mask rows). Synthetic N(0,1) activations and N(0,0.02) weights."""
    import torch
    from fdl import lib, ops
    from fdl.generate import verify_mask
    from fdl.schedule import SeqRows, make_plan

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    bf = lambda *shape, std=1.0: (torch.randn(shape, generator=gen) * std).to(torch.bfloat16).to(dev)  # noqa: E731
    scale = 1.0 / np.sqrt(HD)
    out = {}

    # --- block-table stress
    NB, P = 32, 32
    k_ends = rng.integers(512, 1537, NB)
    full = rng.random(NB) < 0.25
    pages = [(int(k) + P - 1) // P for k in k_ends]
    n_pages = int(sum(pages))
    perm = rng.permutation(n_pages)
    max_pages = max(pages)
    table = np.zeros((NB, max_pages), np.int32)
    nxt = 0
    for b in range(NB):
        table[b, :pages[b]] = perm[nxt:nxt + pages[b]]
        nxt += pages[b]
    n_slots = n_pages * P
    seqs, row, slot_list, logical_list = [], 0, [], []
    for b in range(NB):
        k = int(k_ends[b])
        logical = np.arange(k) if full[b] else None
        if logical is None:
            qn = int(rng.integers(1, 97))
            m = min(qn, 32)
            f = int(rng.integers(96, k - 32 + 1))
            rest = rng.choice(f, qn - m, replace=False) if qn > m else np.zeros(0, np.int64)
            logical = np.concatenate([np.arange(f, f + m), rest])
        logical_list.append(logical)
        slot_list.append(table[b, logical // P].astype(np.int64) * P + logical % P)
        qn = len(logical)
        seqs.append(SeqRows(batch=b, k_end=k, rows=np.arange(row, row + qn), n_imp=min(qn, 32)))
        row += qn
    Q = row
    slots = torch.from_numpy(np.concatenate(slot_list)).to(dev)
    x = bf(Q, D)
    w = [bf(D, D, std=0.02) for _ in range(3)]
    ang = np.outer(np.arange(1536, dtype=np.float32),
                   1.0 / (THETA ** (np.arange(0, HD, 2, dtype=np.float32) / HD)))
    ang = np.concatenate([ang, ang], 1)
    sin = torch.from_numpy(np.sin(ang).astype(np.float32)).to(dev)
    cos = torch.from_numpy(np.cos(ang).astype(np.float32)).to(dev)
    # RoPE at each row's logical position in its sequence
    rope_row = torch.from_numpy(np.concatenate(logical_list).astype(np.int64)).to(dev)
    kc = bf(n_slots, D)
    vc = bf(n_slots, D)
    q = torch.empty((Q, D), dtype=torch.bfloat16, device=dev)
    att = torch.empty_like(q)
    imp = torch.zeros((H, n_slots), dtype=torch.float32, device=dev)
    plan = make_plan(seqs, table, 5, device=dev)
    plan.validate(Q, n_slots)
    t_qkv = _time_op(lambda: ops.qkv_rope_cache(x, *w, sin, cos, slots, q, kc, vc, H,
                                                rope_row=rope_row), reps)
    t_att = _time_op(lambda: ops.block_attention(q, kc, vc, plan, att, H, scale,
                                                 lib.IMP_RAW_LOGIT, imp), reps)
    qk = np.array([len(sq.rows) for sq in seqs], dtype=np.float64)
    kk = k_ends.astype(np.float64)
    f_att = float((4.0 * qk * kk * D).sum())
    b_att = float((2.0 * qk * D * 2 + 2.0 * kk * D * 2).sum())
    f_qkv = 2.0 * Q * D * 3 * D
    out["block_table_stress"] = {
        "workload": f"{NB} sequences, caches 512-1536 keys in permuted 32-slot pages, "
                    f"{int(full.sum())} full recomputes, {Q} query rows, raw-logit importance",
        "qkv_rope_cache": {"us": round(t_qkv, 2), "TFLOP/s": round(f_qkv / t_qkv / 1e6, 1),
                           "mfma_frac": round(f_qkv / t_qkv / 1e6 / PEAK_BF16_TFLOPS, 4)},
        "block_attention": {"us": round(t_att, 2), "TFLOP/s": round(f_att / t_att / 1e6, 1),
                            "GB/s": round(b_att / t_att / 1e3, 1)},
    }
    # full-recompute tiles alone (the MFMA-bound class)
    fseqs = [sq for sq in seqs if len(sq.rows) == sq.k_end]
    if fseqs:
        fplan = make_plan(fseqs, table, 5, device=dev)
        t_full = _time_op(lambda: ops.block_attention(q, kc, vc, fplan, att, H, scale), reps)
        ff = float(sum(4.0 * sq.k_end * sq.k_end * D for sq in fseqs))
        out["block_table_stress"]["full_recompute_attention"] = {
            "sequences": len(fseqs), "us": round(t_full, 2),
            "TFLOP/s": round(ff / t_full / 1e6, 1),
            "mfma_frac": round(ff / t_full / 1e6 / PEAK_BF16_TFLOPS, 4)}

    # --- Flash-Verify
    NV, LC, BMV = 16, 1024, 32
    kv = rng.integers(4, 33, NV)
    rows = 2 * BMV  # mask rows per verify block
    key_pos, vblocks, masks, qslots = [], [], [], []
    k0 = q0 = 0
    for b in range(NV):
        S = int(min(kv[b], BMV))
        cand = b * LC + 512 + np.arange(S)
        keys = np.setdiff1d(b * LC + np.arange(LC), cand)
        key_pos.append(keys)
        vblocks.append([k0, k0 + len(keys), q0, q0 + 2 * S])
        k0 += len(keys)
        q0 += 2 * S
        masks.append(verify_mask(0, S, BMV))
        qslots.append(np.concatenate([cand, cand]))  # draft rows, then mask rows
    QV = q0
    xv = bf(QV, D)
    kcv, vcv = bf(NV * LC, D), bf(NV * LC, D)
    sinv = torch.from_numpy(np.tile(np.sin(ang[:LC]), (NV, 1)).astype(np.float32)).to(dev)
    cosv = torch.from_numpy(np.tile(np.cos(ang[:LC]), (NV, 1)).astype(np.float32)).to(dev)
    qv, k1, v1 = (torch.empty((QV, D), dtype=torch.bfloat16, device=dev) for _ in range(3))
    attv = torch.empty_like(qv)
    kp = torch.from_numpy(np.concatenate(key_pos).astype(np.int64)).to(dev)
    vb = torch.from_numpy(np.array(vblocks, dtype=np.int32)).to(dev)
    mk = torch.from_numpy(np.concatenate(masks).astype(np.uint8)).to(dev)
    qs = torch.from_numpy(np.concatenate(qslots).astype(np.int64)).to(dev)
    t_vq = _time_op(lambda: ops.qkv_rope_cache(xv, *w, sinv, cosv, qs, qv, k1, v1, H,
                                               kv_packed=True), reps)
    t_va = _time_op(lambda: ops.verify_attention(qv, k1, v1, kcv, vcv, kp, vb, mk, rows, attv, H,
                                                 scale), reps)
    sk = np.minimum(kv, BMV).astype(np.float64)
    f_va = float((4.0 * (2 * sk) * (LC - sk + 2 * sk) * D).sum())
    b_va = float((2.0 * (LC - sk) * D * 2 + (LC - sk) * 8 + 2 * (2 * sk) * D * 2).sum())
    out["flash_verify"] = {
        "workload": f"{NV} sequences, 1024-slot caches, {int(sk.sum())} candidates as draft "
                    f"and mask rows ({QV} packed rows)",
        "qkv_rope_cache_packed": {"us": round(t_vq, 2)},
        "verify_attention": {"us": round(t_va, 2), "GB/s": round(b_va / t_va / 1e3, 1),
                             "hbm_frac": round(b_va / t_va / 1e3 / PEAK_HBM_GBS, 4),
                             "TFLOP/s": round(f_va / t_va / 1e6, 1)},
    }
    return out


def run_cpu_baseline(budget_s: float = 15.0, seed: int = 2) -> dict:
    """Times the numpy oracle (one layer of the same workload) on the host cores."""
    from oracle import flash_cache_oracle as orc
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        threads = os.cpu_count() or 1
    host, _ = build_workload(seed, None)
    f32 = lambda t: t.float().numpy()  # noqa: E731
    x, wq, wk, wv = f32(host["x"]), f32(host["wq"]), f32(host["wk"]), f32(host["wv"])
    kc = np.zeros((B * L, D), np.float32)
    vc = np.zeros((B * L, D), np.float32)
    pre = np.concatenate([b * L + np.arange(K_END) for b in range(B)])
    _, kc, vc = orc.qkv_proj_cache(f32(host["x_prefill"]), wq, wk, wv, host["sin"], host["cos"],
                                   pre, H, kc, vc)
    scale = 1.0 / np.sqrt(HD)
    blocks = np.concatenate([host["mb"], host["tb"]])

    def one_layer():
        q, kc2, vc2 = orc.qkv_proj_cache(x, wq, wk, wv, host["sin"], host["cos"], host["slots"], H,
                                         kc, vc)
        orc.block_attention(q, kc2, vc2, blocks, L, H, scale)
        sc = orc.importance_softmax_colsum(q, kc2, host["mb"], B, L, H, scale)
        for b, f in enumerate(host["frontier"]):
            orc.topk(sc, b * L + np.arange(int(f)), TOPK)

    times = []
    t_start = time.perf_counter()
    while True:
        t = time.perf_counter()
        one_layer()
        times.append(time.perf_counter() - t)
        if time.perf_counter() - t_start > budget_s or len(times) >= 5:
            break
    return {"value": float(np.median(times) * 1e6), "unit": "us/layer", "cores": int(threads),
            "kind": "port",
            "sample": f"numpy oracle, {len(times)} full layer(s) of the same workload "
                      f"(QKV+RoPE+cache write, attention, softmax importance, top-32), median; "
                      f"host os.cpu_count()={os.cpu_count()}"}


E2E = dict(batch=8, prompt=256, gen=512, block=32, track_num=1, mask_num=1, threshold=0.9,
           gamma=0.9, verify=True)


def run_e2e(max_steps: int | None, torch_steps: int, seed: int = 0) -> dict:
    """Random-init LLaDA-8B (32 layers, d_model 4096, SiLU-gated MLP 12288, vocab 126464,
    bf16) under the Flash-Cache + Flash-Verify decode loop: batch 8, 256-token random
    prompts, 512 generated tokens, block 32, 32 tracked tokens, verify eps = gamma = 0.9.
    tokens/s = decoded tokens / wall seconds of the decode loop (GPU-synchronised)."""
    import torch
    from flash_cache_hip import flash_fused_elastic_cache
    from fdl.generate import DecodeStats, generate_with_Flash_dLLM
    from fdl.model import LLaDAConfig, build_model
    from fdl.torch_path import flash_fused_elastic_cache_torch

    dev = torch.device("cuda:0")
    cfg = LLaDAConfig.llada_8b()
    model = build_model(cfg, flash_fused_elastic_cache, dev, torch.bfloat16, seed=seed)
    rng = np.random.default_rng(seed)
    n = E2E["batch"]
    prompts = []
    for _ in range(n):
        p = rng.integers(0, cfg.vocab_size, E2E["prompt"])
        p[(p == cfg.mask_token_id) | (p == cfg.eos_token_id)] = 0
        prompts.append(torch.from_numpy(p))
    lengths = [E2E["prompt"]] * n
    kw = dict(gen_length=E2E["gen"], block_length=E2E["block"], mask_id=cfg.mask_token_id,
              threshold=E2E["threshold"], gamma=E2E["gamma"], track_num=E2E["track_num"],
              mask_num=E2E["mask_num"], eos_id=cfg.eos_token_id, verify=E2E["verify"])

    def decode(steps, kv_pages=None):
        st = DecodeStats()
        generate_with_Flash_dLLM(model, prompts, lengths, n, [None] * n, [0] * n, stats=st,
                                 max_steps=steps, kv_pages=kv_pages, **kw)
        return st

    decode(2)  # warm-up: library GEMM selection, allocator
    st = decode(max_steps)
    out = {"tokens_per_s": st.decoded / st.wall_s, "decoded_tokens": st.decoded,
           "steps": st.steps, "forwards": st.forwards, "wall_s": round(st.wall_s, 3),
           "ms_per_step": round(1e3 * st.wall_s / max(st.steps, 1), 3),
           "verify_accepted": st.verify_accepted}
    # the same decode over a paged K/V pool with one fixed stride's worth of pages per row
    stride = ((E2E["prompt"] + E2E["gen"] + E2E["block"]) // 128 + 1) * 128
    stp = decode(max_steps, kv_pages=n * stride // 32)
    out["paged_pool"] = {"tokens_per_s": stp.decoded / stp.wall_s, "steps": stp.steps,
                         "ms_per_step": round(1e3 * stp.wall_s / max(stp.steps, 1), 3),
                         "kv_pages": n * stride // 32}
    if torch_steps > 0:
        model.set_attention(flash_fused_elastic_cache_torch)
        stt = decode(torch_steps)
        model.set_attention(flash_fused_elastic_cache)
        out["torch_gpu"] = {"tokens_per_s": stt.decoded / stt.wall_s, "steps": stt.steps,
                            "ms_per_step": round(1e3 * stt.wall_s / max(stt.steps, 1), 3),
                            "sample": f"first {stt.steps} steps (incl. the full-recompute step 0) "
                                      "of the same decode with the unfused PyTorch driver"}
    del model
    torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description="Flash-Cache hot-path benchmark (one MI355X)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--no-e2e", action="store_true", help="skip the LLaDA-8B decode leg")
    ap.add_argument("--no-torch", action="store_true",
                    help="skip the unfused PyTorch timing of the same layer")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the block-table stress and Flash-Verify measurements")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run five 100 MiB device-to-device copies (the reference kernel for "
                         "scaling the FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--e2e-steps", type=int, default=None,
                    help="bound the HIP decode to this many steps (default: run to completion)")
    ap.add_argument("--e2e-torch-steps", type=int, default=24,
                    help="steps of the unfused PyTorch driver decode (0: skip)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        return 2
    r = run_gpu(args.steps, args.warmup)
    if args.copy_calibration:
        import torch
        src = torch.empty(100 * 1024 * 1024, dtype=torch.uint8, device="cuda:0").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    Q = r["Q"]
    per = r["per_kernel_us"]
    cnt = algorithmic_counts(Q)
    us_layer = r["total_ms"] * 1e3 / args.steps
    qkv_f, qkv_b = cnt["qkv"]
    attn_f, attn_b = cnt["attn"]
    t_qkv, t_attn = per["qkv_rope_cache"], per["block_attention"]
    kernels = {
        "qkv_rope_cache": {"us": t_qkv, "TFLOP/s": qkv_f / t_qkv / 1e6, "GB/s": qkv_b / t_qkv / 1e3,
                           "mfma_frac": qkv_f / t_qkv / 1e6 / PEAK_BF16_TFLOPS},
        "block_attention": {"us": t_attn, "TFLOP/s": attn_f / t_attn / 1e6,
                            "GB/s": attn_b / t_attn / 1e3,
                            "hbm_frac": attn_b / t_attn / 1e3 / PEAK_HBM_GBS},
        "importance_accumulate_rank": {"us": per["importance_accumulate_rank"]},
    }
    achieved = qkv_f / t_qkv / 1e6
    traffic = measured_traffic()
    if "block_attention" in traffic:
        kernels["block_attention"]["traffic_bytes"] = traffic["block_attention"]
    out = {
        "metric": METRIC,
        "value": round(us_layer, 2),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_layer / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) hidden states, N(0,0.02) weights, cache prefilled by the "
                "same fused kernel",
        "config": {"workload": "single layer bf16: batch 8, cache 768 keys (stride 896), block 32, "
                               "32 masked + 32 tracked rows per sequence, softmax-colsum importance, "
                               "top-32",
                   "batch": B, "cache_len": K_END, "q_rows": Q, "d_model": D, "n_heads": H,
                   "head_dim": HD},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic.get("qkv_rope_cache"), "kernel": "qkv_rope_cache",
                     "traffic_source": TRAFFIC_FILE.name},
        "kernels": {k: {kk: round(vv, 3) for kk, vv in v.items()} for k, v in kernels.items()},
    }
    if not args.no_torch:
        tl = run_torch_layer()
        tl["speedup_of_this_build"] = round(tl["us"] / us_layer, 2)
        out["torch_gpu_layer"] = tl
    if not args.no_configs:
        out["configs"] = run_configs()
    if not args.no_e2e:
        out["e2e_llada8b"] = run_e2e(args.e2e_steps, args.e2e_torch_steps)
    if not args.no_cpu:
        out["cpu_baseline"] = run_cpu_baseline(args.cpu_budget)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
