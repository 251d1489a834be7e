"""bench.py's roofline accounting on the CPU: the algorithmic bytes and flops behind
`roofline.achieved`, the committed HBM-traffic summary behind `roofline.traffic`, and the
one-GPU contract of the command line.

The counts are checked against closed forms written out term by term (the cache update:
the three weight matrices once, x, Q and the scattered K / V rows, the sin / cos rows and
the slot indices; the attention: each sequence's query rows in and out, its keys' K and V,
the per-head importance partials) at the sizes where the figures are quoted (118.0 MB and
51.54 GFLOP at 512 rows, 102.0 MB at 40 rows, 109.8 MB for the attention), so a dropped
term or a wrong factor fails here, not only in the bench line."""
import subprocess
import sys

import bench

D, H, HD = 4096, 32, 128


def test_cache_update_counts_at_512_and_40_rows():
    for Q, mb, gf in ((512, 117.968896, 51.539607552), (40, 102.015296, 4.02653184)):
        f, b = bench.algorithmic_counts(Q)["qkv"]
        weights = 3 * D * D * 2
        rows = Q * D * 2 * (1 + 1 + 2)  # x in, Q out, K and V scattered
        rope = Q * HD * 4 * 2            # one sin and one cos row (float32) per row
        index = Q * 8                    # the int64 slot of each row
        assert b == weights + rows + rope + index
        assert abs(b / 1e6 - mb) < 1e-6
        assert f == 2 * Q * D * 3 * D
        assert abs(f / 1e9 - gf) < 1e-6


def test_attention_counts_single_layer():
    f, b = bench.algorithmic_counts(512)["attn"]
    B, rows, keys = bench.B, bench.BM + bench.TRACK, bench.K_END
    assert (B, rows, keys) == (8, 64, 768)
    qo = 2 * rows * D * 2           # the query rows read and the output rows written
    kv = 2 * keys * D * 2           # each key's K and V once per sequence
    partials = keys * H * 4         # the per-head float32 importance partials
    assert b == B * (qo + kv + partials)
    assert abs(b / 1e6 - 109.838336) < 1e-6
    # QK^T and PV over every row, plus the importance pass over the masked rows
    assert f == B * 4 * rows * keys * D + B * 2 * bench.BM * keys * D


def test_committed_traffic_summary_parses():
    t = bench.measured_traffic()
    alg_qkv = bench.algorithmic_counts(512)["qkv"][1]
    alg_attn = bench.algorithmic_counts(512)["attn"][1]
    # measured HBM bytes per launch: at least the algorithmic bytes less the rounding of the
    # counters, and within the re-read factor the summary explains (X once per XCD)
    assert 0.99 * alg_qkv <= t["qkv_rope_cache"] <= 1.4 * alg_qkv
    assert 0.95 * alg_attn <= t["block_attention"] <= 1.1 * alg_attn


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(bench.ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
