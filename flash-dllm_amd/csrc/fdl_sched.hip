// Device-side decode scheduler of the Flash-Cache + Flash-Verify loop (gfx950).
//
// The bookkeeping of llada/generate.py:125-470 kept in device memory, so that a denoising
// step runs its pass-1 forward, the verify forward and the ranking back to back and the host
// synchronises once per step (to learn the next step's row counts and completions):
//   sched_pass1_kernel   pass-1 acceptance (generate.py:215-258 with Flash-Verify,
//                        :335-350 without) and the Flash-Verify lists: fill rows, candidate
//                        draft and mask rows, the key list and the per-block (T, S) of the
//                        closed-form mask (:260-297)
//   sched_verify_kernel  verify acceptance: cumulative product of the mask rows' draft-token
//                        probabilities against gamma (:307-333)
//   sched_pack_kernel    completion test and the next step's masked / tracked lists
//                        (:364-383), packed as the reference packs them (:439-467): masked
//                        rows of every sequence, then tracked rows; plus the attention work
//                        items of that packing
// The ranking itself (:364-366) is fdl_importance_rank / fdl_importance_accumulate_rank on
// the segments the acceptance kernels write.
//
// All three run as one workgroup (the per-step work is a few thousand integers): a wavefront
// per sequence where rows are involved, thread 0 for the prefix sums across sequences.
#include <stdint.h>

#include "fdl_device.h"
#include "fdl_host.h"

namespace fdl {
namespace {

constexpr int kSchedThreads = 256;
constexpr int kSchedWaves = kSchedThreads / kWave;
constexpr int kMaxBm = 128;   // block_m
constexpr int kMaxSeq = 256;  // sequences (batch rows)

struct SchedArgs {
  fdl_sched s;
};

__device__ __forceinline__ int32_t* seq_of(const fdl_sched& s, int j) {
  return s.seq + FDL_SCHED_SEQ_FIELDS * j;
}

// Row k of the pass-1 confidences ranks before row i in the descending sort
// (generate.py:230, :343: x0_p.sort(descending=True), which puts NaN first, as the largest
// value); ties in row order.
__device__ __forceinline__ bool conf_before(double ck, int k, double ci, int i) {
  const bool nk = ck != ck, ni = ci != ci;
  if (nk != ni) return nk;                 // a NaN before a number
  if (nk || ck == ci) return k < i;        // equal (or both NaN): lower row first
  return ck > ci;
}

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}
__device__ __forceinline__ int64_t wave_max(int64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const int64_t o = __shfl_xor(v, off);
    v = o > v ? o : v;
  }
  return v;
}
__device__ __forceinline__ int wave_or(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v |= __shfl_xor(v, off);
  return v;
}

// ------------------------------------------------------------------------------- pass 1
__global__ __launch_bounds__(kSchedThreads) void sched_pass1_kernel(
    fdl_sched s, const double* __restrict__ conf, const int64_t* __restrict__ tok) {
  __shared__ int s_off[kMaxSeq];   // first pass-1 row of sequence j (-1: inactive)
  __shared__ int s_act[kMaxSeq];   // index among the active sequences
  __shared__ int64_t s_koff[kMaxSeq];
  __shared__ double s_c[kSchedWaves][kMaxBm];
  __shared__ int64_t s_p[kSchedWaves][kMaxBm];
  __shared__ int64_t s_t[kSchedWaves][kMaxBm];
  __shared__ int s_dec[kSchedWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int B = static_cast<int>(s.n_seq);
  const int64_t L = s.max_length;
  const int bm = s.block_m;
  if (tid == 0) {
    int acc = 0, na = 0;
    for (int j = 0; j < B; ++j) {
      const int32_t* q = seq_of(s, j);
      if (q[FDL_SEQ_ACTIVE] < 0) {
        s_off[j] = -1;
        s_act[j] = -1;
        continue;
      }
      s_off[j] = acc;
      s_act[j] = na++;
      acc += q[FDL_SEQ_N_MASKED];
    }
  }
  if (lane == 0) s_dec[wave] = 0;
  __syncthreads();
  for (int j = wave; j < B; j += kSchedWaves) {
    if (s_off[j] < 0) continue;
    int32_t* q = seq_of(s, j);
    const int nm = q[FDL_SEQ_N_MASKED], nd0 = q[FDL_SEQ_ND];
    const int64_t eos = q[FDL_SEQ_EOS], pred = q[FDL_SEQ_PRED];
    int64_t* fp = s.full_pos + j * L;
    int n_lmask = 0, n_hi = 0;
    for (int i = lane; i < nm; i += kWave) {
      double c = conf[s_off[j] + i];
      const int64_t p = fp[nd0 + i];
      if (eos != -1 && p >= pred) {  // the predicted-length mask (generate.py:219-225, :339)
        c = 0.0;
        ++n_lmask;
      }
      n_hi += c >= s.threshold;
      s_c[wave][i] = c;
      s_p[wave][i] = p;
      s_t[wave][i] = tok[s_off[j] + i];
    }
    n_lmask = wave_sum(n_lmask);
    n_hi = wave_sum(n_hi);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const int keep = n_hi > 1 ? n_hi : 1;  // at least one token per step
    int64_t ecand = -1;
    for (int i = lane; i < nm; i += kWave) {
      const double ci = s_c[wave][i];
      int rank = 0;
      for (int k = 0; k < nm; ++k) rank += conf_before(s_c[wave][k], k, ci, i);
      const int64_t p = s_p[wave][i], t = s_t[wave][i];
      fp[nd0 + rank] = p;                    // full_pos[nd : nd + nm] = masked[order]
      if (s.verify) s.x_draft[p] = t;        // x_draft[masked] = x0
      if (rank < keep) {
        s.x[p] = t;
        if (t == s.eos_id) ecand = p > ecand ? p : ecand;
      }
    }
    ecand = wave_max(ecand);
    if (lane == 0) {
      const int nd = nd0 + keep;
      q[FDL_SEQ_ND] = nd;
      if (eos == -1 && ecand >= 0) {
        q[FDL_SEQ_EOS] = static_cast<int32_t>(ecand);
        q[FDL_SEQ_PRED] = static_cast<int32_t>(ecand + 1);
      }
      q[FDL_SEQ_KEEP] = keep;
      s_dec[wave] += keep;
      if (!s.verify) {
        s.seg[2 * s_act[j]] = static_cast<int32_t>(j * L);
        s.seg[2 * s_act[j] + 1] = nd - keep;
      } else {
        const int length_num = nm - n_lmask;
        int S = length_num - keep;
        S = S < 0 ? 0 : (S > bm / 2 ? bm / 2 : S);
        int T = 2 * bm - 2 * S;
        if (nd < T) {  // fewer decoded slots than fill rows: raised by the host
          q[FDL_SEQ_ERR] = 1;
          T = nd;
          S = 0;
        }
        q[FDL_SEQ_T] = T;
        q[FDL_SEQ_S] = S;
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    int dec = 0;
    for (int w = 0; w < kSchedWaves; ++w) dec += s_dec[w];
    s.summary[FDL_SUM_DECODED] += dec;
  }
  if (!s.verify) return;
  // Flash-Verify lists: block a (the a-th active sequence) holds rows [2 bm a, 2 bm (a + 1)):
  // T fill rows, S draft rows, S mask rows; its keys are full_pos[:nd - T] and
  // full_pos[nd + S : seqlen_k] (generate.py:272-297).
  if (tid == 0) {
    int64_t koff = 0;
    for (int j = 0; j < B; ++j) {
      if (s_act[j] < 0) continue;
      const int32_t* q = seq_of(s, j);
      const int nd = q[FDL_SEQ_ND], T = q[FDL_SEQ_T], S = q[FDL_SEQ_S], sk = q[FDL_SEQ_SEQLEN_K];
      const int64_t nk1 = nd - T, nk2 = sk - nd - S > 0 ? sk - nd - S : 0;
      const int a = s_act[j];
      s_koff[j] = koff;
      s.vblocks[4 * a] = static_cast<int32_t>(koff);
      s.vblocks[4 * a + 1] = static_cast<int32_t>(koff + nk1 + nk2);
      s.vblocks[4 * a + 2] = 2 * bm * a;
      s.vblocks[4 * a + 3] = 2 * bm * (a + 1);
      s.vmeta[2 * a] = T;
      s.vmeta[2 * a + 1] = S;
      koff += nk1 + nk2;
    }
  }
  __syncthreads();
  for (int j = wave; j < B; j += kSchedWaves) {
    if (s_act[j] < 0) continue;
    const int32_t* q = seq_of(s, j);
    const int nd = q[FDL_SEQ_ND], T = q[FDL_SEQ_T], S = q[FDL_SEQ_S], sk = q[FDL_SEQ_SEQLEN_K];
    const int a = s_act[j];
    const int64_t* fp = s.full_pos + j * L;
    const int64_t r0 = int64_t(2) * bm * a;
    for (int r = lane; r < 2 * bm; r += kWave) {
      // rows: fill full_pos[nd - T + r], drafts and masks of candidate full_pos[nd + i]
      int64_t pos;
      int64_t t;
      if (r < T) {
        pos = fp[nd - T + r];
        t = s.x[pos];
      } else if (r < T + S) {
        pos = fp[nd + r - T];
        t = s.x_draft[pos];
      } else if (r < T + 2 * S) {
        pos = fp[nd + r - T - S];
        t = s.x[pos];
      } else {  // only after a fill-row shortfall (the host raises)
        pos = fp[0];
        t = s.x[pos];
      }
      s.vpos[r0 + r] = pos;
      s.xv[r0 + r] = t;
    }
    const int64_t nk1 = nd - T, nk2 = sk - nd - S > 0 ? sk - nd - S : 0;
    int64_t* kp = s.key_pos + s_koff[j];
    for (int64_t i = lane; i < nk1 + nk2; i += kWave) kp[i] = i < nk1 ? fp[i] : fp[nd + S + (i - nk1)];
    // draft tokens of the last bm / 2 rows of the block (the LM head rows of the verify
    // pass): its mask rows are the last S of them; the others get no token
    const int tail = bm / 2;
    for (int r = lane; r < tail; r += kWave) {
      const int i = r - (tail - S);
      s.draft_tok[int64_t(tail) * a + r] = i >= 0 ? s.x_draft[fp[nd + i]] : -1;
    }
  }
}

// ------------------------------------------------------------------------ verify accept
__global__ __launch_bounds__(kSchedThreads) void sched_verify_kernel(fdl_sched s,
                                                                     const double* __restrict__ prob) {
  __shared__ int s_act[kMaxSeq];
  __shared__ int s_dec;
  const int tid = threadIdx.x;
  const int B = static_cast<int>(s.n_seq);
  const int64_t L = s.max_length;
  const int tail = s.block_m / 2;
  if (tid == 0) {
    int na = 0;
    for (int j = 0; j < B; ++j) s_act[j] = seq_of(s, j)[FDL_SEQ_ACTIVE] < 0 ? -1 : na++;
    s_dec = 0;
  }
  __syncthreads();
  for (int j = tid; j < B; j += kSchedThreads) {
    if (s_act[j] < 0) continue;
    int32_t* q = seq_of(s, j);
    const int a = s_act[j];
    const int S = q[FDL_SEQ_S], nd = q[FDL_SEQ_ND];
    const int64_t eos = q[FDL_SEQ_EOS], pred = q[FDL_SEQ_PRED];
    const int64_t* fp = s.full_pos + j * L;
    // cumprod of the mask rows' draft-token probabilities, left to right (generate.py:318-331)
    double cp = 1.0;
    int keep = 0;
    for (int i = 0; i < S; ++i) {
      double p = prob[int64_t(tail) * a + (tail - S) + i];
      if (eos != -1 && fp[nd + i] >= pred) p = 0.0;
      cp *= p;
      keep += cp >= s.gamma;
    }
    int64_t ecand = -1;
    for (int i = 0; i < keep; ++i) {
      const int64_t pos = fp[nd + i];
      const int64_t t = s.x_draft[pos];
      s.x[pos] = t;
      if (t == s.eos_id) ecand = pos > ecand ? pos : ecand;
    }
    const int ndn = nd + keep;
    q[FDL_SEQ_ND] = ndn;
    q[FDL_SEQ_KEEP] = keep;
    if (eos == -1 && ecand >= 0) {
      q[FDL_SEQ_EOS] = static_cast<int32_t>(ecand);
      q[FDL_SEQ_PRED] = static_cast<int32_t>(ecand + 1);
    }
    s.seg[2 * a] = static_cast<int32_t>(j * L);
    s.seg[2 * a + 1] = ndn - keep;
    atomicAdd(&s_dec, keep);
  }
  __syncthreads();
  if (tid == 0) {
    s.summary[FDL_SUM_DECODED] += s_dec;
    s.summary[FDL_SUM_VERIFY_ACCEPTED] += s_dec;
  }
}

// --------------------------------------------------------------------------------- pack
__global__ __launch_bounds__(kSchedThreads) void sched_pack_kernel(fdl_sched s) {
  __shared__ int s_moff[kMaxSeq], s_toff[kMaxSeq], s_roff[kMaxSeq], s_woff[kMaxSeq];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int B = static_cast<int>(s.n_seq);
  const int64_t L = s.max_length;
  const int bm = s.block_m;
  // completion (generate.py:384: any undecoded position before the predicted length) and the
  // next step's lists (:367-381; a newly admitted sequence recomputes every slot, :125-134)
  for (int j = wave; j < B; j += kSchedWaves) {
    int32_t* q = seq_of(s, j);
    if (q[FDL_SEQ_ACTIVE] < 0) continue;
    const int nd = q[FDL_SEQ_ND], sk = q[FDL_SEQ_SEQLEN_K];
    const bool fresh = q[FDL_SEQ_FRESH] != 0;
    const int64_t pred = q[FDL_SEQ_PRED];
    const int64_t* fp = s.full_pos + j * L;
    int open = 0;
    for (int64_t i = nd + lane; i < L && !open; i += kWave) open |= fp[i] < pred;
    open = wave_or(open);
    const bool done = !fresh && !open;
    int nm = 0, nt = 0, t0 = 0, t1 = 0;
    if (!done) {
      nm = static_cast<int>(L - nd < bm ? L - nd : bm);
      if (fresh || s.track_num < 0) {
        t0 = 0;
        t1 = sk;
      } else {
        t0 = nd - s.track_num * bm > 0 ? nd - s.track_num * bm : 0;
        t1 = nd + bm * s.mask_num < sk ? nd + bm * s.mask_num : sk;
      }
      nt = (nd - t0) + (t1 - (nd + bm) > 0 ? t1 - (nd + bm) : 0);
    }
    // the highest slot the next step's rows query (masked full_pos[nd, nd + nm), tracked
    // full_pos[t0, nd) and [nd + bm, t1)): a paged pool's host grows the row's pages to it
    int64_t hi = -1;
    for (int i = lane; i < nm; i += kWave) hi = fp[nd + i] > hi ? fp[nd + i] : hi;
    for (int i = t0 + lane; i < nd; i += kWave) hi = fp[i] > hi ? fp[i] : hi;
    for (int i = nd + bm + lane; i < t1; i += kWave) hi = fp[i] > hi ? fp[i] : hi;
    hi = wave_max(hi);
    if (lane == 0) {
      q[FDL_SEQ_DONE] = done;
      q[FDL_SEQ_FRESH] = 0;
      q[FDL_SEQ_N_MASKED] = nm;
      q[FDL_SEQ_N_TRACKED] = nt;
      q[FDL_SEQ_T0] = t0;
      q[FDL_SEQ_T1] = t1;
      q[FDL_SEQ_HI] = hi < 0 ? -1 : static_cast<int32_t>(hi - j * L);
    }
  }
  __syncthreads();
  if (tid == 0) {
    // packed rows: masked rows of every sequence, then tracked rows (generate.py:439-467);
    // work items by class (long: more than 128 rows, in 256-row tiles; mid: 65-128; short),
    // each class in sequence order, row lists in the same order as the items
    int acc = 0, n_cont = 0, n_done = 0;
    for (int j = 0; j < B; ++j) {
      const int32_t* q = seq_of(s, j);
      s_moff[j] = acc;
      if (q[FDL_SEQ_ACTIVE] >= 0) {
        acc += q[FDL_SEQ_N_MASKED];
        if (q[FDL_SEQ_DONE]) ++n_done;
        else ++n_cont;
      }
    }
    const int n_masked_rows = acc;
    for (int j = 0; j < B; ++j) {
      const int32_t* q = seq_of(s, j);
      s_toff[j] = acc;
      if (q[FDL_SEQ_ACTIVE] >= 0) acc += q[FDL_SEQ_N_TRACKED];
    }
    int cnt[3] = {0, 0, 0}, rows[3] = {0, 0, 0};
    for (int j = 0; j < B; ++j) {
      const int32_t* q = seq_of(s, j);
      const int n = q[FDL_SEQ_ACTIVE] >= 0 ? q[FDL_SEQ_N_MASKED] + q[FDL_SEQ_N_TRACKED] : 0;
      if (n == 0) continue;
      const int cls = n <= 64 ? 2 : (n <= 128 ? 1 : 0);
      cnt[cls] += cls == 0 ? (n + 255) / 256 : 1;
      rows[cls] += n;
    }
    int wbase[3] = {0, cnt[0], cnt[0] + cnt[1]};
    int rbase[3] = {0, rows[0], rows[0] + rows[1]};
    for (int j = 0; j < B; ++j) {
      const int32_t* q = seq_of(s, j);
      const int n = q[FDL_SEQ_ACTIVE] >= 0 ? q[FDL_SEQ_N_MASKED] + q[FDL_SEQ_N_TRACKED] : 0;
      s_roff[j] = -1;
      if (n == 0) continue;
      const int cls = n <= 64 ? 2 : (n <= 128 ? 1 : 0);
      s_roff[j] = rbase[cls];
      s_woff[j] = wbase[cls];
      rbase[cls] += n;
      wbase[cls] += cls == 0 ? (n + 255) / 256 : 1;
    }
    int32_t* sm = s.summary;
    sm[FDL_SUM_Q] = acc;
    sm[FDL_SUM_N_MASKED_ROWS] = n_masked_rows;
    sm[FDL_SUM_N_LONG] = cnt[0];
    sm[FDL_SUM_N_MID] = cnt[1];
    sm[FDL_SUM_N_SHORT] = cnt[2];
    sm[FDL_SUM_N_CONT] = n_cont;
    sm[FDL_SUM_N_DONE] = n_done;
    sm[FDL_SUM_OVERFLOW] = acc > s.q_cap || cnt[0] + cnt[1] + cnt[2] > s.work_cap;
  }
  __syncthreads();
  if (s.summary[FDL_SUM_OVERFLOW]) return;  // the host raises; nothing is written past a buffer
  for (int j = wave; j < B; j += kSchedWaves) {
    if (s_roff[j] < 0) continue;
    const int32_t* q = seq_of(s, j);
    const int nd = q[FDL_SEQ_ND], nm = q[FDL_SEQ_N_MASKED], nt = q[FDL_SEQ_N_TRACKED];
    const int t0 = q[FDL_SEQ_T0], n1 = nd - t0;
    const int64_t* fp = s.full_pos + j * L;
    for (int i = lane; i < nm; i += kWave) {
      const int64_t p = fp[nd + i];
      s.qpos[s_moff[j] + i] = p;
      s.xq[s_moff[j] + i] = s.x[p];
      s.row_idx[s_roff[j] + i] = s_moff[j] + i;
    }
    for (int i = lane; i < nt; i += kWave) {
      const int64_t p = i < n1 ? fp[t0 + i] : fp[nd + bm + (i - n1)];
      s.qpos[s_toff[j] + i] = p;
      s.xq[s_toff[j] + i] = s.x[p];
      s.row_idx[s_roff[j] + nm + i] = s_toff[j] + i;
    }
    const int n = nm + nt;
    const int chunk = n <= 128 ? n : 256;
    for (int c = lane; c * chunk < n; c += kWave) {
      int32_t* w = s.work + 8 * (s_woff[j] + c);
      const int r0 = c * chunk, nr = n - r0 < chunk ? n - r0 : chunk;
      w[0] = j;
      w[1] = 0;
      w[2] = q[FDL_SEQ_SEQLEN_K];
      w[3] = s_roff[j] + r0;
      w[4] = nr;
      w[5] = c == 0 ? nm : 0;  // the masked rows feed the importance (first tile)
      w[6] = 0;
      w[7] = 0;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Work list from the reference's block tables (fdl_work_from_blocks).
//
// Rows (batch, k_end, q0, q1) of the masked table, then of the tracked table
// (generate.py:52-58, :146-163, :439-465), are grouped by (batch, k_end) in order of first
// appearance; a group's rows are its masked rows (entry order) then its tracked rows, and
// its masked rows are its importance rows. A group of up to 64 rows is one short tile, up
// to 128 one mid tile, more one 256-row tile per 256 rows; tiles go to fixed-capacity
// regions [long | mid | short] of the work array and unused items are zero (no rows, no
// keys: the attention and importance kernels skip them). The same grouping and tile
// classes as fdl.schedule.build_work, without the host: tiles stay in group order within a
// class instead of longest first.
//
// The tables pass through LDS in chunks of kWfbChunk entries, twice: the first pass finds
// the groups and their row counts, the second gives each entry its first row (one cursor
// per group for its masked rows and one for its tracked rows) and writes its row list. Only
// the groups stay in LDS, so the table length is not bounded: a full recompute of 32
// sequences at block_m 16 (generate.py:129-134) has about 1,800-2,800 entries.
constexpr int kWfbChunk = 1024;
constexpr int kWfbMaxGroups = 1024;
constexpr int kWfbMaxSeq = 1024;

struct WfbArgs {
  const int64_t* masked;
  const int64_t* tracked;
  int32_t* work;
  int32_t* row_idx;
  int32_t* status;  // [4]: long, mid, short tiles, error flags (or NULL)
  int n_masked, n_tracked, n_seq;
  int64_t n_q_rows, max_k;
  int cap_long, cap_mid, cap_short;
};

__global__ __launch_bounds__(kSchedThreads) void work_from_blocks_kernel(WfbArgs a) {
  __shared__ int s_ghead[kWfbMaxSeq];                       // newest group of a batch row
  __shared__ int s_gnext[kWfbMaxGroups];                    // next group of the same row
  __shared__ int s_gb[kWfbMaxGroups], s_gk[kWfbMaxGroups];  // group key (batch, k_end)
  __shared__ int s_gm[kWfbMaxGroups], s_gt[kWfbMaxGroups];  // its masked / tracked rows
  __shared__ int s_goff[kWfbMaxGroups];                     // its first row
  __shared__ int s_cm[kWfbMaxGroups], s_ct[kWfbMaxGroups];  // next masked / tracked row
  __shared__ int4 s_e[kWfbChunk];   // a chunk of entries (b, k_end, q0, q1); b = -1: dropped
  __shared__ int s_eoff[kWfbChunk];  // an entry's first row (-1: no rows written)
  __shared__ int s_n_groups, s_err;
  __shared__ int s_used[3];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int n = a.n_masked + a.n_tracked;
  const int max_rows = int(a.n_q_rows);  // < 2^31 (checked by the launcher)
  for (int i = tid; i < a.n_seq; i += kSchedThreads) s_ghead[i] = -1;
  if (tid == 0) {
    s_n_groups = 0;
    s_err = 0;
  }
  // entries [c0, c0 + cnt) into s_e (an entry outside the tables' ranges is dropped)
  auto stage = [&](int c0, int cnt) {
    for (int i = tid; i < cnt; i += kSchedThreads) {
      const int e = c0 + i;
      const int64_t* src = e < a.n_masked ? a.masked + 4 * int64_t(e)
                                          : a.tracked + 4 * int64_t(e - a.n_masked);
      const int64_t b = src[0], k = src[1], q0 = src[2], q1 = src[3];
      const bool ok = b >= 0 && b < a.n_seq && k > 0 && k <= a.max_k && q0 >= 0 && q1 >= q0 &&
                      q1 <= a.n_q_rows;
      s_e[i] = ok ? make_int4(int(b), int(k), int(q0), int(q1)) : make_int4(-1, 0, 0, 0);
    }
  };
  auto lookup = [&](int b, int k) {
    int g = s_ghead[b];
    while (g >= 0 && s_gk[g] != k) g = s_gnext[g];
    return g;
  };
  __syncthreads();
  // pass 1: groups in order of first appearance, with their masked and tracked row counts
  // (saturated past max_rows: such a group gets no tile)
  for (int c0 = 0; c0 < n; c0 += kWfbChunk) {
    const int cnt = min(kWfbChunk, n - c0);
    stage(c0, cnt);
    __syncthreads();
    if (tid == 0) {
      int G = s_n_groups, err = s_err;
      for (int i = 0; i < cnt; ++i) {
        const int4 e = s_e[i];
        if (e.x < 0) {
          err |= 1;
          continue;
        }
        int g = lookup(e.x, e.y);
        if (g < 0) {
          if (G == kWfbMaxGroups) {
            err |= 16;
            continue;
          }
          g = G++;
          s_gb[g] = e.x;
          s_gk[g] = e.y;
          s_gm[g] = s_gt[g] = 0;
          s_gnext[g] = s_ghead[e.x];
          s_ghead[e.x] = g;
        }
        int& c = c0 + i < a.n_masked ? s_gm[g] : s_gt[g];
        c = int(min(int64_t(c) + (e.w - e.z), int64_t(max_rows) + 1));
      }
      s_n_groups = G;
      s_err = err;
    }
    __syncthreads();
  }
  const int G = s_n_groups;
  if (tid == 0) {
    int64_t off = 0;
    for (int g = 0; g < G; ++g) {
      const int o = int(min(off, int64_t(max_rows)));
      s_goff[g] = s_cm[g] = o;
      s_ct[g] = int(min(off + s_gm[g], int64_t(max_rows)));
      off += int64_t(s_gm[g]) + s_gt[g];
    }
    if (off > max_rows) s_err |= 2;
  }
  __syncthreads();
  // pass 2: each entry's first row (a group's masked entries in order, then its tracked
  // ones; an entry whose rows would pass max_rows gets none) and its row list q0 .. q1 - 1
  for (int c0 = 0; c0 < n; c0 += kWfbChunk) {
    const int cnt = min(kWfbChunk, n - c0);
    stage(c0, cnt);
    __syncthreads();
    if (tid == 0) {
      for (int i = 0; i < cnt; ++i) {
        const int4 e = s_e[i];
        const int g = e.x < 0 ? -1 : lookup(e.x, e.y);
        s_eoff[i] = -1;
        if (g < 0) continue;
        int& cur = c0 + i < a.n_masked ? s_cm[g] : s_ct[g];
        if (e.w - e.z > max_rows - cur) continue;  // the group is past max_rows: no tile
        s_eoff[i] = cur;
        cur += e.w - e.z;
      }
    }
    __syncthreads();
    for (int i = wave; i < cnt; i += kSchedWaves) {
      const int o = s_eoff[i];
      if (o < 0) continue;
      const int4 e = s_e[i];
      for (int r = lane; r < e.w - e.z; r += kWave) a.row_idx[o + r] = int32_t(e.z + r);
    }
    __syncthreads();
  }
  if (tid == 0) {
    int err = s_err;
    // tiles, in group order within each class
    int nl = 0, nm = 0, ns = 0;
    for (int g = 0; g < G; ++g) {
      const int64_t rows64 = int64_t(s_gm[g]) + s_gt[g];
      if (rows64 == 0) continue;
      if (s_goff[g] + rows64 > max_rows) {  // rows past max_rows were not written
        err |= 2;
        continue;
      }
      const int rows = int(rows64), start = s_goff[g], n_imp = s_gm[g];
      auto put = [&](int slot, int r0, int nr, int imp) {
        u32x4* w = reinterpret_cast<u32x4*>(a.work + 8 * int64_t(slot));
        w[0] = u32x4{uint32_t(s_gb[g]), 0u, uint32_t(s_gk[g]), uint32_t(r0)};
        w[1] = u32x4{uint32_t(nr), uint32_t(imp), 0u, 0u};
      };
      if (rows <= 64) {
        if (ns < a.cap_short) put(a.cap_long + a.cap_mid + ns, start, rows, n_imp);
        else err |= 4;
        ++ns;
      } else if (rows <= 128) {
        if (nm < a.cap_mid) put(a.cap_long + nm, start, rows, n_imp);
        else err |= 4;
        ++nm;
      } else {
        if (n_imp > 256) err |= 8;  // importance rows beyond one long tile are not counted
        for (int t0 = 0; t0 < rows; t0 += 256) {
          const int nr = min(256, rows - t0);
          if (nl < a.cap_long) put(nl, start + t0, nr, t0 == 0 ? min(n_imp, nr) : 0);
          else err |= 4;
          ++nl;
        }
      }
    }
    s_used[0] = min(nl, a.cap_long);
    s_used[1] = min(nm, a.cap_mid);
    s_used[2] = min(ns, a.cap_short);
    if (a.status) {
      const u32x4 st = {uint32_t(nl), uint32_t(nm), uint32_t(ns), uint32_t(err)};
      *reinterpret_cast<u32x4*>(a.status) = st;
    }
  }
  __syncthreads();
  // unused items of each region: zero (no rows, no keys)
  const int cap[3] = {a.cap_long, a.cap_mid, a.cap_short};
  for (int c = 0, base = 0; c < 3; base += cap[c], ++c)
    for (int i = s_used[c] + tid; i < cap[c]; i += kSchedThreads) {
      u32x4* w = reinterpret_cast<u32x4*>(a.work + 8 * int64_t(base + i));
      w[0] = u32x4{0u, 0u, 0u, 0u};
      w[1] = u32x4{0u, 0u, 0u, 0u};
    }
}

int check_sched(const char* fn, const fdl_sched* s) {
  FDL_REQUIRE(s != nullptr, FDL_ERR_NULL, "%s: state is NULL", fn);
  FDL_REQUIRE(s->n_seq >= 1 && s->n_seq <= kMaxSeq, FDL_ERR_UNSUPPORTED,
              "%s: n_seq = %lld outside [1, %d]", fn, (long long)s->n_seq, kMaxSeq);
  FDL_REQUIRE(s->block_m >= 2 && s->block_m <= kMaxBm, FDL_ERR_UNSUPPORTED,
              "%s: block_m = %d outside [2, %d]", fn, s->block_m, kMaxBm);
  FDL_REQUIRE(s->max_length >= s->block_m && s->n_seq * s->max_length < (int64_t(1) << 31),
              FDL_ERR_SHAPE, "%s: max_length = %lld out of range", fn, (long long)s->max_length);
  FDL_REQUIRE(s->x && s->x_draft && s->full_pos && s->seq && s->summary, FDL_ERR_NULL,
              "%s: a state array is NULL", fn);
  return FDL_OK;
}

}  // namespace
}  // namespace fdl

extern "C" int fdl_sched_pass1(const fdl_sched* state, const double* conf, const int64_t* tok,
                               void* stream) {
  using namespace fdl;
  int rc = check_sched("fdl_sched_pass1", state);
  if (rc != FDL_OK) return rc;
  FDL_REQUIRE(state->seg != nullptr, FDL_ERR_NULL, "fdl_sched_pass1: seg is NULL");
  FDL_REQUIRE(!state->verify || (state->vpos && state->xv && state->key_pos && state->vblocks &&
                                 state->vmeta && state->draft_tok),
              FDL_ERR_NULL, "fdl_sched_pass1: a verify list is NULL");
  hipLaunchKernelGGL(sched_pass1_kernel, dim3(1), dim3(kSchedThreads), 0,
                     static_cast<hipStream_t>(stream), *state, conf, tok);
  FDL_HIP_CHECK(hipGetLastError());
  return ok();
}

extern "C" int fdl_sched_verify_accept(const fdl_sched* state, const double* prob, void* stream) {
  using namespace fdl;
  int rc = check_sched("fdl_sched_verify_accept", state);
  if (rc != FDL_OK) return rc;
  FDL_REQUIRE(state->seg != nullptr && prob != nullptr, FDL_ERR_NULL,
              "fdl_sched_verify_accept: seg or prob is NULL");
  hipLaunchKernelGGL(sched_verify_kernel, dim3(1), dim3(kSchedThreads), 0,
                     static_cast<hipStream_t>(stream), *state, prob);
  FDL_HIP_CHECK(hipGetLastError());
  return ok();
}

extern "C" int fdl_sched_pack(const fdl_sched* state, void* stream) {
  using namespace fdl;
  int rc = check_sched("fdl_sched_pack", state);
  if (rc != FDL_OK) return rc;
  FDL_REQUIRE(state->qpos && state->xq && state->row_idx && state->work, FDL_ERR_NULL,
              "fdl_sched_pack: a step buffer is NULL");
  FDL_REQUIRE(state->q_cap >= 0 && state->work_cap >= 0, FDL_ERR_SHAPE,
              "fdl_sched_pack: q_cap = %lld, work_cap = %lld", (long long)state->q_cap,
              (long long)state->work_cap);
  hipLaunchKernelGGL(sched_pack_kernel, dim3(1), dim3(kSchedThreads), 0,
                     static_cast<hipStream_t>(stream), *state);
  FDL_HIP_CHECK(hipGetLastError());
  return ok();
}

extern "C" int fdl_work_from_blocks(const int64_t* masked, int64_t n_masked, const int64_t* tracked,
                                    int64_t n_tracked, int64_t n_seq, int64_t n_q_rows,
                                    int64_t max_k, int32_t* work, int64_t cap_long,
                                    int64_t cap_mid, int64_t cap_short, int32_t* row_idx,
                                    int32_t* status, void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_masked >= 0 && n_tracked >= 0 && n_masked + n_tracked < (int64_t(1) << 30),
              FDL_ERR_UNSUPPORTED, "fdl_work_from_blocks: %lld table rows (fewer than 2^30)",
              (long long)(n_masked + n_tracked));
  FDL_REQUIRE(n_seq >= 1 && n_seq <= kWfbMaxSeq, FDL_ERR_UNSUPPORTED,
              "fdl_work_from_blocks: n_seq = %lld outside [1, %d]", (long long)n_seq, kWfbMaxSeq);
  FDL_REQUIRE(n_q_rows >= 0 && n_q_rows < (int64_t(1) << 31) && max_k >= 1 &&
                  max_k < (int64_t(1) << 31),
              FDL_ERR_SHAPE, "fdl_work_from_blocks: n_q_rows / max_k out of range");
  FDL_REQUIRE(cap_long >= 0 && cap_mid >= 0 && cap_short >= 0 &&
                  cap_long + cap_mid + cap_short < (int64_t(1) << 30),
              FDL_ERR_SHAPE, "fdl_work_from_blocks: capacities out of range");
  FDL_REQUIRE((n_masked == 0 || masked) && (n_tracked == 0 || tracked), FDL_ERR_NULL,
              "fdl_work_from_blocks: a table is NULL");
  FDL_REQUIRE(work || cap_long + cap_mid + cap_short == 0, FDL_ERR_NULL,
              "fdl_work_from_blocks: work is NULL");
  FDL_REQUIRE(row_idx || n_q_rows == 0, FDL_ERR_NULL, "fdl_work_from_blocks: row_idx is NULL");
  FDL_REQUIRE_ALIGNED(work, 16);
  FDL_REQUIRE_ALIGNED(status, 16);
  WfbArgs a;
  a.masked = masked;
  a.tracked = tracked;
  a.work = work;
  a.row_idx = row_idx;
  a.status = status;
  a.n_masked = int(n_masked);
  a.n_tracked = int(n_tracked);
  a.n_seq = int(n_seq);
  a.n_q_rows = n_q_rows;
  a.max_k = max_k;
  a.cap_long = int(cap_long);
  a.cap_mid = int(cap_mid);
  a.cap_short = int(cap_short);
  hipLaunchKernelGGL(work_from_blocks_kernel, dim3(1), dim3(kSchedThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  FDL_HIP_CHECK(hipGetLastError());
  return ok();
}
