// Pooled-QK scoring, block selection and list compaction.
//
// Restates fpv2/selection.py:109-201 (block_scores_and_select) fused with
// fpv2/kernel.py:141-184 (compact_block_indices).  One workgroup owns one
// (KV head h, query tile t): the tile's G*tile_q packed query rows (head-major:
// row = g*tile_q + p) are scored against the pooled keys with bf16/f16 MFMA
// (S = Q . Kbar^T, fp32 accumulation), each block's energy
//     E_b = sum_{g,rows} exp(s - m),  m = max over fully visible blocks
// is reduced on the fly as (c_b, e_b) = (column max, sum exp(s - c_b)) so
// no [rows, Nb] score tile is ever materialised, then
//     selected = (E_b >= alpha * max_b E_b | sink | local | dense tail) & visible
// and the mask is compacted in LDS into the fixed-width ascending lists
// (selected ascending, then the rest ascending — a stable argsort of -mask),
// with no host synchronisation.
#include "fpv2_common.h"

namespace fpv2 {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerPass = 128;  // 4 waves x 32 rows

struct SelectArgs {
  const void* q;
  const void* pk;
  int64_t G, Hkv, Nt, Nb, Lq_pad, Lq, Lk, offset, bk, tq, sink, window, last_n;
  float scale, alpha;
  int64_t q_hs, q_rs;
  int64_t pk_hs;  // elements between KV heads of pk
  uint8_t* sel_out;
  float* scores;
  int32_t* ids;
  int32_t* counts;
  int32_t* pids;
  int32_t* pcounts;
};

struct TileInfo {
  int64_t h, t, tile_first, tile_last, nfv, nvis;
};

__device__ __forceinline__ TileInfo tile_info(const SelectArgs& a) {
  TileInfo ti;
  const int64_t bid = blockIdx.x;
  ti.h = bid % a.Hkv;
  ti.t = a.Nt - 1 - bid / a.Hkv;  // latest tiles (longest rows) first
  ti.tile_first = a.offset + ti.t * a.tq;
  int64_t last = ti.tile_first + a.tq;
  if (last > a.offset + a.Lq) last = a.offset + a.Lq;
  ti.tile_last = last - 1;
  int64_t nfv = (ti.tile_last + 1) / a.bk;  // blocks with end <= tile_last + 1
  if (nfv > a.Nb) nfv = a.Nb;
  if (nfv < 0) nfv = 0;
  ti.nfv = nfv;
  return ti;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Block-wide max (all threads get the result).  `red` holds >= 4 floats.
__device__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return r;
}
__device__ int block_sum_int(int v, int* red) {
  v = wave_sum_int(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  int r = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return r;
}

// Energies are kept in base 2: logits x = s * log2(e), and a block's running
// (c, e) = (max x, sum 2^(x - c)).  2^(x - m) = exp(s - m / log2(e)), so the
// energies, their ratios and the selection are those of exp(s - max).
constexpr float kLog2e = 1.4426950408889634f;
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Merge (c, e) pairs: sum of 2^(x - c) terms under a common max.
__device__ __forceinline__ void merge_ce(float& c, float& e, float c2, float e2) {
  const float nc = fmaxf(c, c2);
  if (nc == neg_inf()) return;
  const float a = (c == neg_inf()) ? 0.f : e * exp2_fast(c - nc);
  const float b = (c2 == neg_inf()) ? 0.f : e2 * exp2_fast(c2 - nc);
  c = nc;
  e = a + b;
}

// Write one (h, t) row of the two block lists from 0/1 flags (generic
// pointers: LDS or global).  Positions: a selected block goes to the number
// of selected blocks before it; an unselected block goes after all selected
// ones, at total_sel + (#unselected before it).
__device__ void compact_row(const uint8_t* fsel, const uint8_t* fpr, int64_t Nb, int tot_sel,
                            int tot_pr, int32_t* ids, int32_t* pids, int* red) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int run_s = 0, run_p = 0;
  for (int64_t base = 0; base < Nb; base += kThreads) {
    const int64_t b = base + tid;
    const bool in = b < Nb;
    const bool s = in && fsel[b];
    const bool p = in && fpr[b];
    const uint64_t ms = __ballot(s);
    const uint64_t mp = __ballot(p);
    if (lane == 0) {
      red[w] = __popcll(ms);
      red[4 + w] = __popcll(mp);
    }
    __syncthreads();
    int off_s = 0, off_p = 0, sum_s = 0, sum_p = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int cs = red[i], cp = red[4 + i];
      if (i < w) {
        off_s += cs;
        off_p += cp;
      }
      sum_s += cs;
      sum_p += cp;
    }
    __syncthreads();
    if (in) {
      const int ps = run_s + off_s + __popcll(ms & below);  // selected before b
      const int pp = run_p + off_p + __popcll(mp & below);
      const int64_t pos_s = s ? ps : tot_sel + (b - ps);
      const int64_t pos_p = p ? pp : tot_pr + (b - pp);
      ids[pos_s] = static_cast<int32_t>(b);
      pids[pos_p] = static_cast<int32_t>(b);
    }
    run_s += sum_s;
    run_p += sum_p;
  }
}

// Selection rule for block b of tile ti given its energy (selection.py:183-195).
__device__ __forceinline__ bool select_rule(const SelectArgs& a, const TileInfo& ti, int64_t b,
                                            bool energy_ok) {
  const int64_t bs = b * a.bk;
  const int64_t be = bs + a.bk;
  const int64_t tail_from = a.Nt - a.last_n > 0 ? a.Nt - a.last_n : 0;
  const bool forced = bs < a.sink || be > ti.tile_first - a.window || ti.t >= tail_from;
  const bool visible = bs <= ti.tile_last;
  return (energy_ok || forced) && visible;
}

// Shared tail: turn per-block (c_b, e_b) into the mask and lists.
// cb/eb live in LDS and hold valid entries for b < ti.nfv.
__device__ void finish_tile(const SelectArgs& a, const TileInfo& ti, float* cb, float* eb,
                            uint8_t* fsel, uint8_t* fpr, float* fred, int* ired) {
  const int tid = threadIdx.x;
  float m = neg_inf();
  for (int64_t b = tid; b < ti.nfv; b += kThreads) m = fmaxf(m, cb[b]);
  m = block_max(m, fred);
  float emax = 0.f;
  for (int64_t b = tid; b < ti.nfv; b += kThreads) {
    const float c = cb[b];
    const float E = (c == neg_inf()) ? 0.f : eb[b] * exp2_fast(c - m);
    eb[b] = E;
    emax = fmaxf(emax, E);
  }
  emax = block_max(emax, fred);
  const float thr = a.alpha * emax;
  int ns = 0, np = 0;
  for (int64_t b = tid; b < a.Nb; b += kThreads) {
    const float E = (b < ti.nfv) ? eb[b] : 0.f;
    const bool s = select_rule(a, ti, b, E >= thr);
    const int64_t be = (b + 1) * a.bk;
    const bool p = !s && (be < a.Lk ? be : a.Lk) <= ti.tile_first;
    fsel[b] = s;
    fpr[b] = p;
    ns += s;
    np += p;
    if (a.sel_out) a.sel_out[(ti.h * a.Nt + ti.t) * a.Nb + b] = s;
  }
  if (!a.ids) return;
  const int tot_s = block_sum_int(ns, ired);
  const int tot_p = block_sum_int(np, ired);
  __syncthreads();
  const int64_t row = ti.h * a.Nt + ti.t;
  compact_row(fsel, fpr, a.Nb, tot_s, tot_p, a.ids + row * a.Nb, a.pids + row * a.Nb, ired);
  if (tid == 0) {
    a.counts[row] = tot_s;
    a.pcounts[row] = tot_p;
  }
}

// ---------------------------------------------------------------------------
// Score-output path: bf16 / f16 queries and pooled keys, head_dim D (multiple
// of 16), taken when the caller asks for the scores or the scale is not
// positive (the ring path below serves the rest).  Each wave owns 32-block
// chunks of pooled keys in VGPRs and loops over the pass's row groups.
// LDS: Q pass [128][D+8] (reused for the flag arrays), c_b[Nb], e_b[Nb].
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(kThreads, (D <= 128 ? 3 : 2)) void select_mfma_kernel(SelectArgs a) {
  constexpr int LDQ = D + 8;  // padded row: conflict-free 16-byte column reads
  constexpr int KS = D / 16;  // MFMA k-steps over the head dimension
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* qs = reinterpret_cast<uint16_t*>(smem);
  float* cb = reinterpret_cast<float*>(smem + kRowsPerPass * LDQ * 2);
  float* eb = cb + a.Nb;
  __shared__ float fred[4];
  __shared__ int ired[8];
  __shared__ int rpos[kRowsPerPass];  // local query position, -1: no such row
  __shared__ int rhead[kRowsPerPass]; // g of the packed row
  __shared__ int rg_lo[kRowsPerPass / 32], rg_hi[kRowsPerPass / 32];  // per 32-row group

  const TileInfo ti = tile_info(a);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hf = lane >> 5;
  const int64_t R = a.G * a.tq;
  const int64_t n_comp = a.scores ? a.Nb : ti.nfv;
  const uint16_t* pk = static_cast<const uint16_t*>(a.pk) + ti.h * a.pk_hs;
  const uint16_t* qbase = static_cast<const uint16_t*>(a.q);
  const float sc2 = a.scale * kLog2e;
  const bool fast_ok = a.scores == nullptr && sc2 > 0.f;

  for (int64_t b = tid; b < n_comp; b += kThreads) {
    cb[b] = neg_inf();
    eb[b] = 0.f;
  }

  for (int64_t rc = 0; rc < R; rc += kRowsPerPass) {
    __syncthreads();
    if (tid < kRowsPerPass) {
      const int64_t pr = rc + tid;
      int p = -1, gg = 0;
      if (pr < R) {
        gg = static_cast<int>(pr / a.tq);
        p = static_cast<int>(ti.t * a.tq + (pr - gg * a.tq));
      }
      rpos[tid] = p;
      rhead[tid] = gg;
    }
    __syncthreads();
    // Lowest and highest position of each 32-row group (-1 rows make the
    // group take the checked path).
    if (tid < kRowsPerPass / 32) {
      int lo_p = 0x7fffffff, hi_p = -1;
      for (int r = 0; r < 32; ++r) {
        const int p = rpos[tid * 32 + r];
        lo_p = min(lo_p, p);
        hi_p = max(hi_p, p);
      }
      rg_lo[tid] = lo_p;
      rg_hi[tid] = hi_p;
    }
    // Stage 128 packed rows of Q (zeros past the tile or the valid length).
    // For D <= 128 each thread issues all its loads before the stores, so the
    // staging costs one memory round trip instead of one per load (D = 256
    // keeps one load at a time: its registers hold no more across the pass).
    constexpr int QN = kRowsPerPass * (D / 8) / kThreads;
    static_assert(kRowsPerPass * (D / 8) % kThreads == 0, "Q staging splits evenly");
    constexpr int QB = D <= 128 ? QN : 1;
#pragma unroll 1
    for (int i0 = 0; i0 < QN; i0 += QB) {
      u32x4 qst[QB];
#pragma unroll
      for (int i = 0; i < QB; ++i) {
        const int e = tid + (i0 + i) * kThreads;
        const int r = e / (D / 8);
        const int c = e - r * (D / 8);
        const int64_t pr = rc + r;
        qst[i] = u32x4{0u, 0u, 0u, 0u};
        if (pr < R) {
          const int64_t g = pr / a.tq;
          const int64_t pos = ti.t * a.tq + (pr - g * a.tq);
          if (pos < a.Lq) qst[i] = load16(qbase + (ti.h * a.G + g) * a.q_hs + pos * a.q_rs + c * 8);
        }
      }
#pragma unroll
      for (int i = 0; i < QB; ++i) {
        const int e = tid + (i0 + i) * kThreads;
        const int r = e / (D / 8);
        store16(qs + r * LDQ + (e - r * (D / 8)) * 8, qst[i]);
      }
    }
    __syncthreads();
    const int64_t rows_here = (R - rc) < kRowsPerPass ? (R - rc) : kRowsPerPass;
    const int nrg = static_cast<int>((rows_here + 31) / 32);
    // Lowest / highest row position of the pass (wave-uniform).
    int pass_lo = 0x7fffffff, pass_hi = -1;
    for (int rg = 0; rg < nrg; ++rg) {
      pass_lo = min(pass_lo, rg_lo[rg]);
      pass_hi = max(pass_hi, rg_hi[rg]);
    }
    const int lq = static_cast<int>(a.Lq);

    for (int64_t chunk = wave; chunk * 32 < n_comp; chunk += 4) {
      const int64_t b = chunk * 32 + l32;
      // Rows see block b (fully visible blocks only) from local position lo.
      const bool b_scored = b < ti.nfv;
      int64_t lo64 = b * a.bk - a.offset;
      const int lo = lo64 < 0 ? 0 : static_cast<int>(lo64 > 0x7fffffff ? 0x7fffffff : lo64);
      typename Elem<T>::vec8 kf[KS];
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (b < a.Nb) v = load16(pk + b * D + k * 16 + hf * 8);
        kf[k] = as_vec8<T>(v);
      }
      float cmax = neg_inf(), esum = 0.f;
      // Fast path: every row of the pass sees the lane's block in every lane
      // (the chunks before the diagonal), no scores requested, positive
      // scale: no per-row tests.  The next row group's Q fragments are read
      // from LDS while the current group's energies are summed.
      const bool all_ok = b_scored && pass_lo >= lo && pass_hi < lq;
      if (fast_ok && __ballot(!all_ok) == 0ull) {
        u32x4 qv[2][KS];
#pragma unroll
        for (int k = 0; k < KS; ++k) qv[0][k] = load16(qs + l32 * LDQ + k * 16 + hf * 8);
        for (int rg = 0; rg < nrg; rg += 2) {
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int g = rg + half;
            if (g < nrg) {
              f32x16 acc = {};
#pragma unroll
              for (int k = 0; k < KS; ++k) acc = Elem<T>::mfma32(as_vec8<T>(qv[half][k]), kf[k], acc);
              if (g + 1 < nrg) {
#pragma unroll
                for (int k = 0; k < KS; ++k)
                  qv[half ^ 1][k] = load16(qs + ((g + 1) * 32 + l32) * LDQ + k * 16 + hf * 8);
              }
              float mx = acc[0];
#pragma unroll
              for (int j = 1; j < 16; ++j) mx = fmaxf(mx, acc[j]);
              const float nc = fmaxf(cmax, mx * sc2);
              float e0 = (cmax == neg_inf()) ? 0.f : esum * exp2_fast(cmax - nc), e1 = 0.f;
#pragma unroll
              for (int j = 0; j < 16; j += 2) {
                e0 += exp2_fast(fmaf(acc[j], sc2, -nc));
                e1 += exp2_fast(fmaf(acc[j + 1], sc2, -nc));
              }
              cmax = nc;
              esum = e0 + e1;
            }
          }
        }
      } else {
      for (int rg = 0; rg < nrg; ++rg) {
        f32x16 acc = {};
#pragma unroll
        for (int k = 0; k < KS; ++k) {
          const u32x4 qv = load16(qs + (rg * 32 + l32) * LDQ + k * 16 + hf * 8);
          acc = Elem<T>::mfma32(as_vec8<T>(qv), kf[k], acc);
        }
        // Lane holds rows rg*32 + (j/4)*8 + hf*4 + j%4 of block b.
        float s[16];
        bool ok[16];
        float lm = neg_inf();
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int r = rg * 32 + (j >> 2) * 8 + hf * 4 + (j & 3);
          const int pos = rpos[r];
          if (a.scores && pos >= 0 && b < a.Nb)
            a.scores[((ti.h * a.G + rhead[r]) * a.Lq_pad + pos) * a.Nb + b] = acc[j] * a.scale;
          s[j] = acc[j] * sc2;
          const bool valid = b_scored && pos >= lo && pos < lq;
          ok[j] = valid;
          if (valid) lm = fmaxf(lm, s[j]);
        }
        if (lm != neg_inf()) {
          const float nc = fmaxf(cmax, lm);
          float e = (cmax == neg_inf()) ? 0.f : esum * exp2_fast(cmax - nc);
#pragma unroll
          for (int j = 0; j < 16; ++j)
            if (ok[j]) e += exp2_fast(s[j] - nc);
          cmax = nc;
          esum = e;
        }
      }
      }  // checked path
      // Partner lane (hf ^ 1) holds the other 16 rows of each row group.
      const float oc = __shfl_xor(cmax, 32);
      const float oe = __shfl_xor(esum, 32);
      merge_ce(cmax, esum, oc, oe);
      if (hf == 0 && b < n_comp) {
        float c = cb[b], e = eb[b];
        merge_ce(c, e, cmax, esum);
        cb[b] = c;
        eb[b] = e;
      }
    }
  }
  __syncthreads();
  // The Q staging area is free now: reuse it for the flag arrays.
  uint8_t* fsel = reinterpret_cast<uint8_t*>(smem);
  uint8_t* fpr = fsel + a.Nb;
  finish_tile(a, ti, cb, eb, fsel, fpr, fred, ired);
}

// ---------------------------------------------------------------------------
// Ring path: bf16 / f16, head_dim D (multiple of 16), positive scale, no
// score output -- the hook's path.  Wave w owns the 32 packed rows
// [32w, 32w + 32) of each 128-row pass, its Q fragments in VGPRs.  The pooled
// keys stream through an LDS ring of 32-block chunks filled by
// buffer_load_dwordx4 ... lds kAhead chunks ahead, so the workgroup reads each
// chunk from L2 once and no wave waits on a global load in the loop.  Every
// wave multiplies every chunk (S = Q . Kbar^T, a lane holds 16 rows of one
// block) and sums its rows' 2^(x - m_w) per block against a lazily updated
// wave reference m_w (x = s*log2(e)); one wave adds the four waves' partials
// into the block energies E_b one chunk later, each partial scaled by
// 2^(m_w - G) for the workgroup reference G.  Energies are only compared
// with each other (E_b >= alpha * max E), so any common reference gives the
// same selection as exp(s - max) (selection.py:178-185).
// LDS (dynamic only, so that the ring starts at LDS address 0 and its rows
// are aligned for the XOR-swizzled reads): ring [kRing][32][ROWB], E_b[Nb],
// partials [2 slots][4 waves][32 blocks], their references [2][4], G, row
// positions [128], reduction scratch.
// ---------------------------------------------------------------------------
template <int D>
struct RingGeom {
  static constexpr int ROWB = D <= 64 ? 128 : (D <= 128 ? 256 : 512);  // LDS row (power of two)
  static constexpr int RC = ROWB / 16;      // 16-byte chunks per LDS row
  static constexpr int DG = D / 8;          // chunks holding data
  static constexpr int TILE = 32 * ROWB;    // one 32-block chunk
  static constexpr int NF = TILE / 1024 / (kThreads / 64);  // fill instructions per wave per chunk
  static_assert(TILE % (1024 * (kThreads / 64)) == 0, "fills split evenly over the waves");
  // 16-byte chunk c of row r is stored at chunk c ^ kmask(r): the 16 rows of
  // a ds_read_b128 quarter-wave then hit 16 different 16-byte bank groups
  static __device__ __forceinline__ int kmask(int row) {
    return ROWB >= 256 ? (row & 15) : ((row >> 1) & 7);
  }
};
#ifndef FPV2_SEL_AHEAD
#define FPV2_SEL_AHEAD 2
#endif
constexpr int kAhead = FPV2_SEL_AHEAD;  // chunks filled ahead of the multiply
constexpr int kRing = kAhead + 1;   // ring stages
// A wave's reference m_w is raised only when a chunk's logit exceeds it by
// more than kWaveSlack (log2 units), and G only when some m_w exceeds it by
// more than kGroupSlack: a partial is at most 32 * 2^kWaveSlack and its
// merge factor at most 2^kGroupSlack, far inside float32.
constexpr float kWaveSlack = 16.f;
constexpr float kGroupSlack = 30.f;

template <int D>
constexpr size_t ring_lds_bytes(int64_t Nb) {
  return static_cast<size_t>(kRing) * RingGeom<D>::TILE + static_cast<size_t>(Nb) * 4 +
         (2 * 4 * 32 + 2 * 4 + 4) * 4 + kRowsPerPass * 4 + 16 * 4;
}

__device__ __forceinline__ float wave_max_any(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Mask and lists from the block energies (selection.py:183-195 and
// kernel.py:141-184) in 32-bit arithmetic (the host routes geometries whose
// key positions need more bits elsewhere).  Wave w compacts the blocks
// [w * span, (w + 1) * span) 64 at a time with ballots: one pass counts, the
// waves' counts are exchanged through LDS, a second pass writes each block's
// positions (selected ascending, then the rest ascending; likewise pruned).
__device__ void finish_ring(const SelectArgs& a, int h, int t, int tile_first, int tile_last,
                            int nfv, const float* eb, float* fred, int* ired) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int Nb = static_cast<int>(a.Nb);
  float emax = 0.f;
  for (int b = tid; b < nfv; b += kThreads) emax = fmaxf(emax, eb[b]);
  emax = block_max(emax, fred);
  const float thr = a.alpha * emax;
  const int bk = static_cast<int>(a.bk);
  const int sink = static_cast<int>(a.sink);
  const int first_minus_window = tile_first - static_cast<int>(a.window);
  const int lk = static_cast<int>(a.Lk);
  const bool tail = t >= a.Nt - a.last_n;
  // branch-free: every lane reads an E_b (clamped index; entries past nfv
  // are discarded), so no LDS read is left pending in a divergent branch
  auto flags = [&](int b, bool& sel, bool& pru) {
    const float e_raw = eb[min(b, Nb - 1)];
    const float E = b < nfv ? e_raw : 0.f;
    const int bs = b * bk;
    const int be = bs + bk;
    const bool forced = bs < sink || be > first_minus_window || tail;
    sel = (E >= thr || forced) && bs <= tile_last;
    pru = !sel && min(be, lk) <= tile_first;
  };
  const int span = ((Nb + 4 * 64 - 1) / (4 * 64)) * 64;
  const int w0 = min(Nb, wave * span), w1 = min(Nb, w0 + span);
  int ns = 0, np = 0;
  for (int base = w0; base < w1; base += 64) {
    const int b = base + lane;
    bool sel, pru;
    flags(b, sel, pru);
    sel = sel && b < w1;
    pru = pru && b < w1;
    ns += __popcll(__ballot(sel));
    np += __popcll(__ballot(pru));
  }
  if (lane == 0) {
    ired[wave] = ns;
    ired[4 + wave] = np;
  }
  __syncthreads();
  int run_s = 0, run_p = 0, tot_s = 0, tot_p = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int cs = ired[w], cp = ired[4 + w];
    run_s += w < wave ? cs : 0;
    run_p += w < wave ? cp : 0;
    tot_s += cs;
    tot_p += cp;
  }
  const int64_t row = static_cast<int64_t>(h) * a.Nt + t;
  int32_t* ids = a.ids + row * a.Nb;
  int32_t* pids = a.pids + row * a.Nb;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int base = w0; base < w1; base += 64) {
    const int b = base + lane;
    bool sel, pru;
    flags(b, sel, pru);
    sel = sel && b < w1;
    pru = pru && b < w1;
    const uint64_t ms = __ballot(sel);
    const uint64_t mp = __ballot(pru);
    if (b < w1) {
      const int ps = run_s + __popcll(ms & below);  // selected before b
      const int pp = run_p + __popcll(mp & below);
      ids[sel ? ps : tot_s + (b - ps)] = b;
      pids[pru ? pp : tot_p + (b - pp)] = b;
      if (a.sel_out) a.sel_out[row * a.Nb + b] = sel;
    }
    run_s += __popcll(ms);
    run_p += __popcll(mp);
  }
  if (tid == 0) {
    a.counts[row] = tot_s;
    a.pcounts[row] = tot_p;
  }
}

template <typename T, int D>
__global__ __launch_bounds__(kThreads, (D <= 128 ? 3 : 2)) void select_ring_kernel(SelectArgs a) {
  using GM = RingGeom<D>;
  using vec8 = typename Elem<T>::vec8;
  constexpr int KS = D / 16;  // MFMA k-steps over the head dimension
  extern __shared__ __align__(1024) unsigned char smem[];
  constexpr size_t kRingBytes = static_cast<size_t>(kRing) * GM::TILE;
  float* eb = reinterpret_cast<float*>(smem + kRingBytes);  // block energies, reference G
  float* xe = eb + a.Nb;     // [2 slots][4 waves][32 blocks] chunk partials
  float* xm = xe + 256;      // [2 slots][4 waves] their wave references
  float* gref = xm + 8;      // G
  int* rpos = reinterpret_cast<int*>(gref + 4);  // local query position, -1: no such row
  float* fred = reinterpret_cast<float*>(rpos + kRowsPerPass);
  int* ired = reinterpret_cast<int*>(fred + 4);

  const TileInfo ti = tile_info(a);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hf = lane >> 5;
  const int64_t R = a.G * a.tq;
  const int nfv = static_cast<int>(ti.nfv);
  const int nchunks = (nfv + 31) / 32;
  const float sc2 = a.scale * kLog2e;  // > 0 on this path
  const int lq = static_cast<int>(a.Lq);
  const int offset = static_cast<int>(a.offset);
  const int bk = static_cast<int>(a.bk);

  for (int b = tid; b < nfv; b += kThreads) eb[b] = 0.f;
  if (tid == 0) *gref = neg_inf();

  // ---- fills: chunk c of the pooled keys into ring stage c % kRing ----
  // Fill instruction i of this wave covers LDS bytes [1024 j, 1024 (j + 1))
  // of the stage, j = wave + 4 i: lane -> row (64 j + lane) / RC, stored
  // chunk p = (64 j + lane) % RC, holding data chunk p ^ kmask(row).  Blocks
  // past nfv and pad chunks past D load zeros.
  const rsrc_t pkr = make_rsrc(static_cast<const uint16_t*>(a.pk) + ti.h * a.pk_hs,
                               static_cast<uint32_t>(a.Nb * D * 2));
  int fill_off[GM::NF];  // byte offset within the chunk's 32 rows (-1: pad)
  int fill_row[GM::NF];
#pragma unroll
  for (int i = 0; i < GM::NF; ++i) {
    const int e = 64 * (wave + 4 * i) + lane;
    const int row = e / GM::RC;
    const int c = (e % GM::RC) ^ GM::kmask(row);
    fill_row[i] = row;
    fill_off[i] = c < GM::DG ? (row * D + c * 8) * 2 : -1;
  }
  auto fill_chunk = [&](int c) {
    typedef __attribute__((address_space(3))) void* lds_ptr;
    uint8_t* const sp = smem + (c % kRing) * GM::TILE;
#pragma unroll
    for (int i = 0; i < GM::NF; ++i) {
      const bool ok = c < nchunks && c * 32 + fill_row[i] < nfv && fill_off[i] >= 0;
      const uint32_t off = ok ? static_cast<uint32_t>(c * 32 * D * 2 + fill_off[i]) : kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(pkr, (lds_ptr)(sp + (wave + 4 * i) * 1024), 16, off, 0, 0, 0);
    }
  };
  // K fragment k of the lane's block row l32 (data chunk 2k + hf)
  const uint32_t kread = (lds_addr(smem) + l32 * GM::ROWB + ((16 * hf) ^ (16 * GM::kmask(l32))));

  // add the four waves' partials of chunk c (slot c & 1) to E_b (lanes 0-31
  // of wave c & 3); G follows the largest wave reference with a slack, and
  // the energies merged so far are rescaled when it moves (rare)
  auto merge_chunk = [&](int c) {
    if (lane < 32 && wave == (c & 3)) {
      const float* xms = xm + (c & 1) * 4;
      const float m0 = xms[0], m1 = xms[1], m2 = xms[2], m3 = xms[3];
      const float mc = fmaxf(fmaxf(m0, m1), fmaxf(m2, m3));
      float g = *gref;
      if (mc > g + kGroupSlack) {  // uniform over the merging lanes
        const float f = (g == neg_inf()) ? 0.f : exp2_fast(g - mc);
        for (int b = lane; b < nfv; b += 32) eb[b] *= f;
        g = mc;
        if (lane == 0) *gref = g;
      }
      const int b = c * 32 + lane;
      if (b < nfv) {
        const float* xc = xe + (c & 1) * 128 + lane;
        float e = eb[b];
        if (m0 != neg_inf()) e = fmaf(xc[0], exp2_fast(m0 - g), e);
        if (m1 != neg_inf()) e = fmaf(xc[32], exp2_fast(m1 - g), e);
        if (m2 != neg_inf()) e = fmaf(xc[64], exp2_fast(m2 - g), e);
        if (m3 != neg_inf()) e = fmaf(xc[96], exp2_fast(m3 - g), e);
        eb[b] = e;
      }
    }
  };

  float mref = neg_inf();    // wave reference m_w (log2 units, wave-uniform)
  float thr_raw = neg_inf(); // raw score above which m_w must move: (m_w + slack) / sc2
  for (int64_t rc = 0; rc < R; rc += kRowsPerPass) {
    __syncthreads();  // the previous pass is done with the ring and rpos
    if (tid < kRowsPerPass) {
      const int64_t pr = rc + tid;
      int p = -1;
      if (pr < R) {
        const int64_t gg = pr / a.tq;
        p = static_cast<int>(ti.t * a.tq + (pr - gg * a.tq));
      }
      rpos[tid] = p;
    }
    // this wave's Q fragments: row rc + 32 wave + l32, data chunks 2k + hf
    vec8 qf[KS];
    int my_pos = -1;
    {
      const int64_t pr = rc + wave * 32 + l32;
      const uint16_t* qrow = nullptr;
      if (pr < R) {
        const int64_t g = pr / a.tq;
        const int64_t pos = ti.t * a.tq + (pr - g * a.tq);
        my_pos = static_cast<int>(pos);
        if (pos < a.Lq) qrow = static_cast<const uint16_t*>(a.q) + (ti.h * a.G + g) * a.q_hs + pos * a.q_rs;
      }
#pragma unroll
      for (int k = 0; k < KS; ++k)
        qf[k] = as_vec8<T>(qrow ? load16(qrow + k * 16 + hf * 8) : u32x4{0u, 0u, 0u, 0u});
    }
    // lowest / highest position of the wave's rows (-1 rows force the checked path)
    int g_lo = my_pos, g_hi = my_pos;
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) {
      g_lo = min(g_lo, __shfl_xor(g_lo, o));
      g_hi = max(g_hi, __shfl_xor(g_hi, o));
    }
#pragma unroll
    for (int c = 0; c < kAhead; ++c) fill_chunk(c);

    for (int c = 0; c < nchunks; ++c) {
      vm_wait<GM::NF * (kAhead - 1)>();
      __syncthreads();  // chunk c in LDS; chunk c-1's stage and partial slot are free
      fill_chunk(c + kAhead);
      // S = Q . Kbar^T over the chunk: 8 reads in flight, MFMA k after read k
      const uint32_t ka = kread + (c % kRing) * GM::TILE;
      u32x4 kf[KS];
      StaticFor<0, KS>::run([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        kf[k] = lds_read_b128<true, 0>(ka ^ (32 * k));
      });
      f32x16 acc = {};
      StaticFor<0, KS>::run([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        constexpr int younger = KS - 1 - k < 15 ? KS - 1 - k : 15;
        lgkm_wait<true, younger>(kf[k]);
        acc = Elem<T>::mfma32(qf[k], as_vec8<T>(kf[k]), acc);
      });
      // the previous chunk's merge runs while the MFMAs are in flight
      if (c > 0) merge_chunk(c - 1);
      // Lane holds rows (j/4)*8 + hf*4 + j%4 of the wave's 32 rows, block b.
      const int b = c * 32 + l32;
      const bool b_scored = b < nfv;
      const int lo = max(0, b * bk - offset);
      float e = 0.f;
      if (__ballot(!(b_scored && g_lo >= lo && g_hi < lq)) == 0ull) {
        // every row sees the block: no per-row tests
        float lm = fmaxf(fmaxf(acc[0], acc[1]), acc[2]);
#pragma unroll
        for (int j = 3; j < 15; j += 2) lm = fmaxf(fmaxf(lm, acc[j]), acc[j + 1]);
        lm = fmaxf(lm, acc[15]);
        if (__ballot(lm > thr_raw) != 0ull) {  // rare: raise the wave reference
          mref = wave_max_any(lm) * sc2;
          thr_raw = (mref + kWaveSlack) / sc2;
        }
        const float bias = -mref;
        float e0 = 0.f, e1 = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j += 2) {
          e0 += exp2_fast(fmaf(acc[j], sc2, bias));
          e1 += exp2_fast(fmaf(acc[j + 1], sc2, bias));
        }
        e = e0 + e1;
      } else {
        bool ok[16];
        float lm = neg_inf();
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int pos = rpos[wave * 32 + (j >> 2) * 8 + hf * 4 + (j & 3)];
          ok[j] = b_scored && pos >= lo && pos < lq;
          if (ok[j]) lm = fmaxf(lm, acc[j]);
        }
        if (__ballot(lm > thr_raw) != 0ull) {
          mref = wave_max_any(lm) * sc2;
          thr_raw = (mref + kWaveSlack) / sc2;
        }
        const float bias = -mref;
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (ok[j]) e += exp2_fast(fmaf(acc[j], sc2, bias));
      }
      // partner lane (hf ^ 1) holds the other 16 rows of the block
      {
        const auto es = __builtin_amdgcn_permlane32_swap(__float_as_uint(e), __float_as_uint(e), false, false);
        e = __uint_as_float(es[0]) + __uint_as_float(es[1]);
      }
      if (hf == 0) xe[(c & 1) * 128 + wave * 32 + l32] = e;
      if (lane == 0) xm[(c & 1) * 4 + wave] = mref;
    }
    vm_wait<0>();  // the fills past the last chunk
    __syncthreads();
    if (nchunks > 0) merge_chunk(nchunks - 1);
  }
  __syncthreads();
  finish_ring(a, static_cast<int>(ti.h), static_cast<int>(ti.t), static_cast<int>(ti.tile_first),
              static_cast<int>(ti.tile_last), nfv, eb, fred, ired);
}

// ---------------------------------------------------------------------------
// Generic path (float32 inputs, or head dims without an MFMA instantiation).
// LDS: Q pass [32][D] float, c_b[Nb], e_b[Nb], flags[2*Nb].
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float ld(const void* p, int64_t i);
template <> __device__ __forceinline__ float ld<float>(const void* p, int64_t i) {
  return static_cast<const float*>(p)[i];
}
template <> __device__ __forceinline__ float ld<bf16_t>(const void* p, int64_t i) {
  return Elem<bf16_t>::to_float(static_cast<const uint16_t*>(p)[i]);
}
template <> __device__ __forceinline__ float ld<f16_t>(const void* p, int64_t i) {
  return Elem<f16_t>::to_float(static_cast<const uint16_t*>(p)[i]);
}

constexpr int kGenericRows = 32;

template <typename T>
__global__ __launch_bounds__(kThreads) void select_generic_kernel(SelectArgs a, int D) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* qs = reinterpret_cast<float*>(smem);
  float* cb = qs + kGenericRows * D;
  float* eb = cb + a.Nb;
  uint8_t* fsel = reinterpret_cast<uint8_t*>(eb + a.Nb);
  uint8_t* fpr = fsel + a.Nb;
  __shared__ float fred[4];
  __shared__ int ired[8];
  const TileInfo ti = tile_info(a);
  const int tid = threadIdx.x;
  const int64_t R = a.G * a.tq;
  const int64_t n_comp = a.scores ? a.Nb : ti.nfv;
  for (int64_t b = tid; b < n_comp; b += kThreads) {
    cb[b] = neg_inf();
    eb[b] = 0.f;
  }
  for (int64_t rc = 0; rc < R; rc += kGenericRows) {
    __syncthreads();
    for (int e = tid; e < kGenericRows * D; e += kThreads) {
      const int r = e / D;
      const int d = e - r * D;
      const int64_t pr = rc + r;
      float v = 0.f;
      if (pr < R) {
        const int64_t g = pr / a.tq;
        const int64_t pos = ti.t * a.tq + (pr - g * a.tq);
        if (pos < a.Lq) v = ld<T>(a.q, (ti.h * a.G + g) * a.q_hs + pos * a.q_rs + d);
      }
      qs[e] = v;
    }
    __syncthreads();
    for (int64_t b = tid; b < n_comp; b += kThreads) {
      float c = cb[b], e = eb[b];
      for (int r = 0; r < kGenericRows && rc + r < R; ++r) {
        const int64_t pr = rc + r;
        float dot = 0.f;
        for (int d = 0; d < D; ++d) dot = fmaf(qs[r * D + d], ld<T>(a.pk, ti.h * a.pk_hs + b * D + d), dot);
        const float s = dot * a.scale;
        const int64_t g = pr / a.tq;
        const int64_t pos = ti.t * a.tq + (pr - g * a.tq);
        if (a.scores) a.scores[((ti.h * a.G + g) * a.Lq_pad + pos) * a.Nb + b] = s;
        if (pos < a.Lq && b < ti.nfv && b * a.bk <= a.offset + pos) merge_ce(c, e, s * kLog2e, 1.f);
      }
      cb[b] = c;
      eb[b] = e;
    }
  }
  __syncthreads();
  finish_tile(a, ti, cb, eb, fsel, fpr, fred, ired);
}

// ---------------------------------------------------------------------------
// Standalone compaction of a caller-provided mask (kernel.py:141-184).
// ---------------------------------------------------------------------------
struct CompactArgs {
  const uint8_t* mask;
  int64_t Hkv, Nt, Nb, tq, bk, offset, Lk;
  int32_t *ids, *counts, *pids, *pcounts;
};

__global__ __launch_bounds__(kThreads) void compact_kernel(CompactArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint8_t* fsel = smem;
  uint8_t* fpr = smem + a.Nb;
  __shared__ int ired[8];
  const int64_t row = blockIdx.x;
  const int64_t t = row % a.Nt;
  const int64_t tile_first = a.offset + t * a.tq;
  const uint8_t* m = a.mask + row * a.Nb;
  int ns = 0, np = 0;
  for (int64_t b = threadIdx.x; b < a.Nb; b += kThreads) {
    const bool s = m[b] != 0;
    const int64_t be = (b + 1) * a.bk;
    const bool p = !s && (be < a.Lk ? be : a.Lk) <= tile_first;
    fsel[b] = s;
    fpr[b] = p;
    ns += s;
    np += p;
  }
  const int tot_s = block_sum_int(ns, ired);
  const int tot_p = block_sum_int(np, ired);
  __syncthreads();
  compact_row(fsel, fpr, a.Nb, tot_s, tot_p, a.ids + row * a.Nb, a.pids + row * a.Nb, ired);
  if (threadIdx.x == 0) {
    a.counts[row] = tot_s;
    a.pcounts[row] = tot_p;
  }
}

template <typename K>
int launch_with_lds(K kernel, dim3 grid, size_t lds, hipStream_t stream, const SelectArgs& a) {
  if (lds > 160 * 1024) return fail(FPV2_ERR_UNSUPPORTED, "score_select: %zu bytes of LDS exceed 160 KiB", lds);
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(lds)) != hipSuccess)
    return fail(FPV2_ERR_LAUNCH, "score_select: hipFuncSetAttribute failed");
  hipLaunchKernelGGL(kernel, grid, dim3(kThreads), lds, stream, a);
  return check_launch("score_select");
}

template <typename K>
int launch_generic(K kernel, dim3 grid, size_t lds, hipStream_t stream, const SelectArgs& a, int D) {
  if (lds > 160 * 1024) return fail(FPV2_ERR_UNSUPPORTED, "score_select: %zu bytes of LDS exceed 160 KiB", lds);
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(lds)) != hipSuccess)
    return fail(FPV2_ERR_LAUNCH, "score_select: hipFuncSetAttribute failed");
  hipLaunchKernelGGL(kernel, grid, dim3(kThreads), lds, stream, a, D);
  return check_launch("score_select");
}

template <typename T>
int dispatch_mfma(int64_t D, dim3 grid, hipStream_t stream, const SelectArgs& a, bool* done) {
  *done = true;
  // the ring kernel keeps key positions and list entries in 32 bits
  const bool small = a.Nb * a.bk <= (1LL << 30) && a.offset + a.Lq_pad <= (1LL << 30) &&
                     a.sink <= (1LL << 30) && a.window <= (1LL << 30) && a.Nt <= (1LL << 30);
  if (a.scores == nullptr && a.scale > 0.f && a.ids != nullptr && small) {
    switch (D) {
      case 64: return launch_with_lds(select_ring_kernel<T, 64>, grid, ring_lds_bytes<64>(a.Nb), stream, a);
      case 96: return launch_with_lds(select_ring_kernel<T, 96>, grid, ring_lds_bytes<96>(a.Nb), stream, a);
      case 128: return launch_with_lds(select_ring_kernel<T, 128>, grid, ring_lds_bytes<128>(a.Nb), stream, a);
      case 256: return launch_with_lds(select_ring_kernel<T, 256>, grid, ring_lds_bytes<256>(a.Nb), stream, a);
      default: break;
    }
  }
  const size_t tail = static_cast<size_t>(a.Nb) * 8;
  switch (D) {
    case 64: return launch_with_lds(select_mfma_kernel<T, 64>, grid, 128 * 72 * 2 + tail, stream, a);
    case 96: return launch_with_lds(select_mfma_kernel<T, 96>, grid, 128 * 104 * 2 + tail, stream, a);
    case 128: return launch_with_lds(select_mfma_kernel<T, 128>, grid, 128 * 136 * 2 + tail, stream, a);
    case 256: return launch_with_lds(select_mfma_kernel<T, 256>, grid, 128 * 264 * 2 + tail, stream, a);
    default: *done = false; return 0;
  }
}

}  // namespace
}  // namespace fpv2

extern "C" int fpv2_score_select(const void* q, const void* pooled_k, int dtype,
                                 const fpv2_select_params* p, uint8_t* selected, float* scores,
                                 int32_t* selected_ids, int32_t* selected_counts,
                                 int32_t* pruned_ids, int32_t* pruned_counts, void* stream) {
  using namespace fpv2;
  if (!p || !q || !pooled_k) return fail(FPV2_ERR_ARGUMENT, "score_select: null argument");
  if (p->kv_heads <= 0 || p->query_heads <= 0 || p->query_heads % p->kv_heads)
    return fail(FPV2_ERR_ARGUMENT, "query heads must be divisible by KV heads");
  if (p->head_dim <= 0 || p->block_k <= 0 || p->tile_q <= 0 || p->num_blocks <= 0)
    return fail(FPV2_ERR_ARGUMENT, "score_select: head_dim, block_k, tile_q and num_blocks must be positive");
  if (p->padded_query_length <= 0 || p->padded_query_length % p->tile_q)
    return fail(FPV2_ERR_ARGUMENT, "query length must be padded to a multiple of tile_q");
  if (p->query_length <= 0 || p->query_length > p->padded_query_length)
    return fail(FPV2_ERR_ARGUMENT, "query_length must be in (0, q.shape[-2]]");
  if (p->offset < 0) return fail(FPV2_ERR_ARGUMENT, "offset must be non-negative");
  if (p->offset + p->query_length > p->num_blocks * p->block_k)
    return fail(FPV2_ERR_ARGUMENT, "queries extend beyond the represented key sequence");
  if (p->num_blocks > FPV2_MAX_BLOCKS)
    return fail(FPV2_ERR_UNSUPPORTED, "score_select: num_blocks %lld exceeds %d",
                static_cast<long long>(p->num_blocks), FPV2_MAX_BLOCKS);
  const bool any_list = selected_ids || selected_counts || pruned_ids || pruned_counts;
  const bool all_list = selected_ids && selected_counts && pruned_ids && pruned_counts;
  if (any_list && !all_list) return fail(FPV2_ERR_ARGUMENT, "score_select: give all four list outputs or none");
  if (any_list && (p->key_length <= 0 || p->key_length > p->num_blocks * p->block_k))
    return fail(FPV2_ERR_ARGUMENT, "key_length is inconsistent with selected blocks");
  if (p->pooled_head_stride < p->num_blocks * p->head_dim)
    return fail(FPV2_ERR_ARGUMENT, "score_select: pooled_head_stride must be >= num_blocks*head_dim");
  SelectArgs a{};
  a.q = q;
  a.pk = pooled_k;
  a.Hkv = p->kv_heads;
  a.G = p->query_heads / p->kv_heads;
  a.Lq_pad = p->padded_query_length;
  a.Nt = p->padded_query_length / p->tile_q;
  a.Nb = p->num_blocks;
  a.Lq = p->query_length;
  a.Lk = p->key_length;
  a.offset = p->offset;
  a.bk = p->block_k;
  a.tq = p->tile_q;
  a.sink = p->sink_tokens;
  a.window = p->window_tokens;
  a.last_n = p->last_n_blocks;
  a.scale = p->scale;
  a.alpha = p->alpha;
  a.q_hs = p->q_head_stride;
  a.q_rs = p->q_row_stride;
  a.pk_hs = p->pooled_head_stride;
  a.sel_out = selected;
  a.scores = scores;
  a.ids = selected_ids;
  a.counts = selected_counts;
  a.pids = pruned_ids;
  a.pcounts = pruned_counts;
  const int64_t wgs = a.Hkv * a.Nt;
  if (wgs > 0x7fffffffLL) return fail(FPV2_ERR_UNSUPPORTED, "score_select: grid too large");
  dim3 grid(static_cast<unsigned>(wgs));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t D = p->head_dim;
  const bool vec_ok = D % 8 == 0 && a.q_rs % 8 == 0 && a.q_hs % 8 == 0 && a.pk_hs % 8 == 0 &&
                      reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(pooled_k) % 16 == 0;
  bool done = false;
  int rc = 0;
  if (dtype == FPV2_BF16 && vec_ok) rc = dispatch_mfma<bf16_t>(D, grid, s, a, &done);
  else if (dtype == FPV2_F16 && vec_ok) rc = dispatch_mfma<f16_t>(D, grid, s, a, &done);
  if (done) return rc;
  const size_t lds = static_cast<size_t>(kGenericRows) * D * 4 + static_cast<size_t>(a.Nb) * 10;
  switch (dtype) {
    case FPV2_F32: return launch_generic(select_generic_kernel<float>, grid, lds, s, a, static_cast<int>(D));
    case FPV2_BF16: return launch_generic(select_generic_kernel<bf16_t>, grid, lds, s, a, static_cast<int>(D));
    case FPV2_F16: return launch_generic(select_generic_kernel<f16_t>, grid, lds, s, a, static_cast<int>(D));
    default: return fail(FPV2_ERR_UNSUPPORTED, "score_select: unsupported dtype %d", dtype);
  }
}

extern "C" int fpv2_compact_block_indices(const uint8_t* selected, int64_t kv_heads,
                                          int64_t num_tiles, int64_t num_blocks, int64_t tile_q,
                                          int64_t block_k, int64_t offset, int64_t key_length,
                                          int32_t* selected_ids, int32_t* selected_counts,
                                          int32_t* pruned_ids, int32_t* pruned_counts,
                                          void* stream) {
  using namespace fpv2;
  if (!selected || !selected_ids || !selected_counts || !pruned_ids || !pruned_counts)
    return fail(FPV2_ERR_ARGUMENT, "compact: null argument");
  if (kv_heads <= 0 || num_tiles <= 0 || num_blocks <= 0 || tile_q <= 0 || block_k <= 0)
    return fail(FPV2_ERR_ARGUMENT, "compact: sizes must be positive");
  if (offset < 0) return fail(FPV2_ERR_ARGUMENT, "offset must be non-negative");
  if (key_length <= 0 || key_length > num_blocks * block_k)
    return fail(FPV2_ERR_ARGUMENT, "key_length is inconsistent with selected blocks");
  if (num_blocks * 2 > 160 * 1024) return fail(FPV2_ERR_UNSUPPORTED, "compact: too many blocks");
  CompactArgs a{};
  a.mask = selected;
  a.Hkv = kv_heads;
  a.Nt = num_tiles;
  a.Nb = num_blocks;
  a.tq = tile_q;
  a.bk = block_k;
  a.offset = offset;
  a.Lk = key_length;
  a.ids = selected_ids;
  a.counts = selected_counts;
  a.pids = pruned_ids;
  a.pcounts = pruned_counts;
  const int64_t rows = kv_heads * num_tiles;
  if (rows > 0x7fffffffLL) return fail(FPV2_ERR_UNSUPPORTED, "compact: grid too large");
  const size_t lds = static_cast<size_t>(num_blocks) * 2;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(compact_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(lds)) != hipSuccess)
    return fail(FPV2_ERR_LAUNCH, "compact: hipFuncSetAttribute failed");
  hipLaunchKernelGGL(compact_kernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), lds,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("compact");
}
