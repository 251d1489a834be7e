"""Pins the numpy oracle (oracle/flash_cache_oracle.py) against closed forms, library
routines and brute force, so that a dropped term, a wrong sign or index, or a transposed
operand in the oracle fails here. CPU only."""
import math

import numpy as np
import pytest
import torch

from oracle import flash_cache_oracle as orc

F32 = np.float32


def _bf16_np(shape, gen, std=1.0):
    t = (torch.randn(shape, generator=gen) * std).to(torch.bfloat16)
    return t.float().numpy()


# ----------------------------------------------------------------------------- RoPE

def test_rope_tables_closed_form():
    sin, cos = orc.rope_tables(1024, 128, 500000.0)
    assert sin.dtype == F32 and sin.shape == (1024, 128)
    inv = 1.0 / (500000.0 ** (np.arange(0, 128, 2, dtype=np.float64) / 128))
    ang = np.arange(1024, dtype=np.float64)[:, None] * inv[None, :]
    ang = np.concatenate([ang, ang], axis=1)
    # fp32 argument rounding bounds the error by ~|angle| * 2^-23
    tol = 2e-7 * np.maximum(1.0, np.abs(ang)) + 1e-6
    assert np.all(np.abs(sin - np.sin(ang)) <= tol)
    assert np.all(np.abs(cos - np.cos(ang)) <= tol)
    # position 0 is the identity rotation; both halves share frequencies bit for bit
    assert np.all(sin[0] == 0) and np.all(cos[0] == 1)
    assert np.array_equal(sin[:, :64], sin[:, 64:]) and np.array_equal(cos[:, :64], cos[:, 64:])


def _rope_complex(t, pos, theta, hd):
    """RoPE as complex rotation of (t_c, t_{c+half}) by angle pos * inv_freq_c, float64."""
    half = hd // 2
    inv = 1.0 / (theta ** (np.arange(0, hd, 2, dtype=np.float64) / hd))
    z = t[:, :half].astype(np.float64) + 1j * t[:, half:].astype(np.float64)
    z = z * np.exp(1j * pos[:, None].astype(np.float64) * inv[None, :])
    return np.concatenate([z.real, z.imag], axis=1)


def test_qkv_proj_cache_vs_complex_rotation():
    gen = torch.Generator().manual_seed(1)
    n_heads, hd, Q, L = 2, 128, 10, 64
    D = n_heads * hd
    x = _bf16_np((Q, D), gen)
    wq, wk, wv = (_bf16_np((D, D), gen, 0.02) for _ in range(3))
    sin, cos = orc.rope_tables(L, hd, 10000.0)
    pos = np.array([0, 1, 5, 17, 33, 40, 41, 50, 62, 63], dtype=np.int64)
    kc = np.full((L, D), 7.0, F32)
    vc = np.full((L, D), -3.0, F32)
    q, kc2, vc2 = orc.qkv_proj_cache(x, wq, wk, wv, sin, cos, pos, n_heads, kc, vc)
    x64 = x.astype(np.float64)
    for h in range(n_heads):
        cols = slice(h * hd, (h + 1) * hd)
        q_ref = _rope_complex(x64 @ wq.astype(np.float64).T[:, cols], pos, 10000.0, hd)
        k_ref = _rope_complex(x64 @ wk.astype(np.float64).T[:, cols], pos, 10000.0, hd)
        np.testing.assert_allclose(q[:, cols], q_ref, atol=2e-5, rtol=1e-4)
        np.testing.assert_allclose(kc2[pos][:, cols], k_ref, atol=2e-5, rtol=1e-4)
    np.testing.assert_allclose(vc2[pos], x64 @ wv.astype(np.float64).T, atol=2e-5, rtol=1e-4)
    untouched = np.setdiff1d(np.arange(L), pos)
    assert np.all(kc2[untouched] == 7.0) and np.all(vc2[untouched] == -3.0)
    # position 0 is unrotated
    np.testing.assert_allclose(q[0], (x64 @ wq.astype(np.float64).T)[0], atol=2e-5, rtol=1e-4)


def test_rope_relative_position_and_norm():
    gen = torch.Generator().manual_seed(2)
    hd = 128
    sin, cos = orc.rope_tables(600, hd, 500000.0)
    a = _bf16_np((1, hd), gen)
    b = _bf16_np((1, hd), gen)
    def rot(t, p):
        return orc.rotate_pairs(t, sin[[p]], cos[[p]]).astype(np.float64)
    # per-pair norms are preserved
    ra = rot(a, 77)
    np.testing.assert_allclose(ra[:, :64] ** 2 + ra[:, 64:] ** 2, a[:, :64].astype(np.float64) ** 2 + a[:, 64:] ** 2, rtol=1e-5, atol=1e-6)
    # <R_m a, R_n b> depends only on m - n
    d1 = float((rot(a, 100) * rot(b, 30)).sum())
    d2 = float((rot(a, 570) * rot(b, 500)).sum())
    assert abs(d1 - d2) < 2e-3 * max(1.0, abs(d1))


# ------------------------------------------------------------------------ attention

def _sdpa(q, k, v, n_heads, scale, allow=None):
    """torch's scaled_dot_product_attention on [rows, D] float32 arrays, per head."""
    hd = q.shape[1] // n_heads
    qt = torch.from_numpy(q).view(-1, n_heads, hd).transpose(0, 1).double()
    kt = torch.from_numpy(k).view(-1, n_heads, hd).transpose(0, 1).double()
    vt = torch.from_numpy(v).view(-1, n_heads, hd).transpose(0, 1).double()
    m = None if allow is None else torch.from_numpy(allow)
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=m, scale=scale)
    return o.transpose(0, 1).reshape(-1, n_heads * hd).numpy()


def test_block_attention_vs_sdpa():
    gen = torch.Generator().manual_seed(3)
    n_heads, hd, B, L = 2, 128, 2, 128
    D = n_heads * hd
    kc = _bf16_np((B * L, D), gen)
    vc = _bf16_np((B * L, D), gen)
    q = _bf16_np((20, D), gen)
    blocks = np.array([[0, 100, 0, 7], [1, 128, 7, 20]])
    scale = orc.softmax_scale(hd)
    out = orc.block_attention(q, kc, vc, blocks, L, n_heads, scale)
    np.testing.assert_allclose(out[0:7], _sdpa(q[0:7], kc[:100], vc[:100], n_heads, scale), atol=1e-5)
    np.testing.assert_allclose(out[7:20], _sdpa(q[7:20], kc[L:2 * L], vc[L:2 * L], n_heads, scale), atol=1e-5)


def test_block_attention_paged_equals_contiguous():
    gen = torch.Generator().manual_seed(4)
    n_heads, hd, B, L, P = 1, 128, 2, 128, 32
    D = n_heads * hd
    kc = _bf16_np((B * L, D), gen)
    vc = _bf16_np((B * L, D), gen)
    q = _bf16_np((9, D), gen)
    blocks = np.array([[0, 96, 0, 4], [1, 128, 4, 9]])
    out = orc.block_attention(q, kc, vc, blocks, L, n_heads, 0.1)
    perm = np.random.default_rng(0).permutation(B * L // P)
    # physical page perm[i] holds logical page i: move the data accordingly
    kp = np.zeros_like(kc)
    vp = np.zeros_like(vc)
    table = np.zeros((B, L // P), np.int64)
    for b in range(B):
        for p in range(L // P):
            phys = perm[b * (L // P) + p]
            table[b, p] = phys
            kp[phys * P:(phys + 1) * P] = kc[b * L + p * P: b * L + (p + 1) * P]
            vp[phys * P:(phys + 1) * P] = vc[b * L + p * P: b * L + (p + 1) * P]
    out_p = orc.block_attention(q, kp, vp, blocks, L, n_heads, 0.1, page_table=table, page_size=P)
    np.testing.assert_array_equal(out, out_p)


def test_attention_closed_forms():
    gen = torch.Generator().manual_seed(5)
    D = 128
    q = _bf16_np((3, D), gen)
    v = _bf16_np((5, D), gen)
    # one key: output is that key's value
    k1 = _bf16_np((1, D), gen)
    np.testing.assert_allclose(orc.attend(q, k1, v[:1], 1, 0.3), np.repeat(v[:1], 3, 0), atol=1e-6)
    # identical keys: output is the mean of the values
    ks = np.repeat(k1, 5, axis=0)
    np.testing.assert_allclose(orc.attend(q, ks, v, 1, 0.3), np.repeat(v.mean(0, keepdims=True), 3, 0), atol=1e-5)
    # masked-out keys have no effect
    allow = np.ones((3, 5), bool)
    allow[:, 3:] = False
    np.testing.assert_allclose(orc.attend(q, _bf16_np((5, D), gen) * 0 + ks, v, 1, 0.3, allow),
                               np.repeat(v[:3].mean(0, keepdims=True), 3, 0), atol=1e-5)


def test_importance_raw_closed_form():
    gen = torch.Generator().manual_seed(6)
    n_heads, hd, B, L, bm = 2, 128, 2, 128, 4
    D = n_heads * hd
    kc = _bf16_np((B * L, D), gen)
    q = _bf16_np((8, D), gen)
    masked = np.array([[0, 96, 0, 4], [1, 128, 4, 8]])
    S = orc.importance_raw_S(q, kc, masked, B, L, n_heads, bm)
    scores = orc.importance_accumulate(np.zeros(B * L, F32), S)
    # mean over (rows, heads) of q_r^h . k_n^h = (sum_r q_r) . k_n / (bm * H) over full D
    exp = np.zeros(B * L)
    for b, k_end, q0, q1 in masked:
        qs = q[q0:q1].astype(np.float64).sum(0)
        exp[b * L: b * L + k_end] = kc[b * L: b * L + k_end].astype(np.float64) @ qs / (bm * n_heads)
    np.testing.assert_allclose(scores, exp, atol=1e-4, rtol=1e-4)
    assert np.all(scores[96:L] == 0)


def test_importance_softmax_colsum_vs_torch_softmax():
    gen = torch.Generator().manual_seed(7)
    n_heads, hd, B, L = 2, 128, 1, 128
    D = n_heads * hd
    kc = _bf16_np((B * L, D), gen)
    q = _bf16_np((4, D), gen)
    scale = orc.softmax_scale(hd)
    got = orc.importance_softmax_colsum(q, kc, np.array([[0, 100, 0, 4]]), B, L, n_heads, scale)
    exp = np.zeros(L)
    for h in range(n_heads):
        s = torch.from_numpy(q[:, h * hd:(h + 1) * hd]).double() @ torch.from_numpy(kc[:100, h * hd:(h + 1) * hd]).double().T
        exp[:100] += torch.softmax(s * scale, dim=1).sum(0).numpy()
    np.testing.assert_allclose(got, exp, atol=1e-5)
    assert abs(got.sum() - 4 * n_heads) < 1e-4  # each row's probabilities sum to one


def test_importance_f64_raw_exact_sum():
    """float64 raw importance = the exact mean of every product q_r^h[d] k_n^h[d] (math.fsum
    is exactly rounded), ragged blocks counting block_m rows, keys past k_end untouched."""
    import math
    gen = torch.Generator().manual_seed(16)
    n_heads, hd, B, L, bm = 3, 128, 2, 64, 4
    D = n_heads * hd
    kc = _bf16_np((B * L, D), gen)
    q = _bf16_np((7, D), gen)
    masked = np.array([[0, 40, 0, 4], [1, 64, 4, 7]])  # the second block has 3 of 4 rows
    got = orc.importance_f64(q, kc, masked, B, L, n_heads, "raw", 0.0, bm)
    for b, k_end, q0, q1 in masked:
        for n in (0, 5, k_end - 1):
            terms = [float(q[r, d]) * float(kc[b * L + n, d]) for r in range(q0, q1) for d in range(D)]
            assert abs(got[b * L + n] - math.fsum(terms) / (bm * n_heads)) <= 1e-12 * (1 + abs(got[b * L + n]))
    assert np.all(got[40:L] == 0)


def test_importance_f64_softmax_vs_torch_float64():
    gen = torch.Generator().manual_seed(17)
    n_heads, hd, B, L = 2, 128, 2, 64
    D = n_heads * hd
    kc = _bf16_np((B * L, D), gen)
    q = _bf16_np((6, D), gen)
    scale = orc.softmax_scale(hd)
    masked = np.array([[0, 50, 0, 3], [1, 64, 3, 6]])
    got = orc.importance_f64(q, kc, masked, B, L, n_heads, "softmax", scale, 32)
    exp = np.zeros(B * L)
    for b, k_end, q0, q1 in masked:
        for h in range(n_heads):
            cols = slice(h * hd, (h + 1) * hd)
            s = torch.from_numpy(q[q0:q1, cols]).double() @ torch.from_numpy(kc[b * L:b * L + k_end, cols]).double().T
            exp[b * L:b * L + k_end] += torch.softmax(s * scale, dim=1).sum(0).numpy()
    np.testing.assert_allclose(got, exp, rtol=1e-13, atol=1e-15)
    # each row's probabilities sum to one, for every head
    assert abs(got.sum() - 6 * n_heads) < 1e-12


# --------------------------------------------------------------------------- verify

def test_verify_mask_kat_T2_S3():
    bm = 4
    m = orc.verify_mask(2, 3, bm)
    T, F = True, False
    exp = np.array([
        # fill fill  d0 d1 d2   m0 m1 m2
        [T, T, F, F, F, T, T, T],   # fill rows never see drafts (:268)
        [T, T, F, F, F, T, T, T],
        [T, T, T, F, F, F, T, T],   # draft i: drafts j <= i (m11), masks j > i (m12)
        [T, T, T, T, F, F, F, T],
        [T, T, T, T, T, F, F, F],
        [T, T, F, F, F, T, T, T],   # mask i: drafts j < i (m21), masks j >= i (m22)
        [T, T, T, F, F, F, T, T],
        [T, T, T, T, F, F, F, T],
    ])
    np.testing.assert_array_equal(m, exp)
    # no row sees its own draft: draft row T+i and mask row T+S+i vs column T+i
    for i in range(3):
        assert not m[2 + 3 + i, 2 + i]


def test_verify_mask_kat_no_fill():
    m = orc.verify_mask(0, 2, 2)
    T, F = True, False
    np.testing.assert_array_equal(m, np.array([
        [T, F, F, T],
        [T, T, F, F],
        [F, F, T, T],
        [T, F, F, T],
    ]))


def test_verify_attention_vs_sdpa():
    gen = torch.Generator().manual_seed(8)
    n_heads, hd, bm = 2, 128, 4
    D = n_heads * hd
    n_slots = 64
    kc = _bf16_np((n_slots, D), gen)
    vc = _bf16_np((n_slots, D), gen)
    rows = 2 * bm
    q = _bf16_np((2 * rows, D), gen)
    k1 = _bf16_np((2 * rows, D), gen)
    v1 = _bf16_np((2 * rows, D), gen)
    key_pos = np.array([3, 9, 10, 11, 40, 41, 2, 60, 61], dtype=np.int64)
    vblocks = np.array([[0, 5, 0, rows], [5, 9, rows, 2 * rows]], dtype=np.int32)
    mask = np.concatenate([orc.verify_mask(2, 3, bm), orc.verify_mask(0, 4, bm)], axis=0)
    scale = orc.softmax_scale(hd)
    out = orc.verify_attention(q, k1, v1, kc, vc, key_pos, mask, vblocks, rows, n_heads, scale)
    for v, (k0, kk1, q0, q1) in enumerate(vblocks):
        keys = np.concatenate([kc[key_pos[k0:kk1]], k1[q0:q1]])
        vals = np.concatenate([vc[key_pos[k0:kk1]], v1[q0:q1]])
        allow = np.concatenate([np.ones((rows, kk1 - k0), bool), mask[v * rows:(v + 1) * rows]], axis=1)
        np.testing.assert_allclose(out[q0:q1], _sdpa(q[q0:q1], keys, vals, n_heads, scale, allow), atol=1e-5)


# --------------------------------------------------------------------------- top-k

def test_rank_and_topk_brute_force():
    rng = np.random.default_rng(9)
    scores = rng.integers(-3, 4, size=200).astype(F32) * F32(0.5)  # many ties
    scores[5] = -0.0
    scores[6] = 0.0
    slots = rng.permutation(200)[:150].astype(np.int64)
    asc = orc.rank_ascending(scores, slots)
    brute = sorted(slots.tolist(), key=lambda s: (float(scores[s]) + 0.0, -s))
    assert asc.tolist() == brute
    top = orc.topk(scores, slots, 10)
    brute_top = sorted(slots.tolist(), key=lambda s: (-(float(scores[s]) + 0.0), s))[:10]
    assert top.tolist() == brute_top
    short = orc.topk(scores, slots[:3], 5)
    assert short[3:].tolist() == [-1, -1]


# ------------------------------------------------------------------------- schedule

def test_make_blocks_kat():
    t = orc.make_blocks(1, [512, 896], 40, 110, 32)
    np.testing.assert_array_equal(t, [[1, 896, 40, 72], [1, 896, 72, 104], [1, 896, 104, 110]])


def test_layout_kat():
    # prompt 128 + gen 256 with block 32: L = ((128 + 256 + 32) // 128 + 1) * 128 = 512
    assert orc.max_length_for([128], 256, 32) == 512
    assert orc.seqlen_k_for(128, 256) == 512
    # prompt 256 + gen 512 + block 32 -> L = 896, k_end = 896
    assert orc.max_length_for([256], 512, 32) == 896
    assert orc.seqlen_k_for(256, 512) == 896
    assert math.isclose(orc.softmax_scale(128), 1 / math.sqrt(128))
