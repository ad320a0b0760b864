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
  uint32_t tq_magic;  // ceil(2^32 / tq), streaming path
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
// positive (the streaming and owner paths below serve the rest).  Each wave owns 32-block
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
// Shared by the hook's paths (bf16 / f16, head_dim a multiple of 16, positive
// scale, no score output).  Block energies are sums of 2^(x - m_w), x =
// s * log2(e), against a lazily raised per-wave reference m_w, rescaled to a
// common reference before the selection.  Energies are only compared with
// each other (E_b >= alpha * max E), so any common reference gives the same
// selection as exp(s - max) (selection.py:178-185).
// ---------------------------------------------------------------------------
// A wave's reference m_w is raised only when a logit exceeds it by more than
// kWaveSlack (log2 units): a row group's sum is at most 16 * 2^kWaveSlack
// per lane, far inside float32.
constexpr float kWaveSlack = 16.f;

__device__ __forceinline__ float wave_max_any(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// The same without LDS traffic: DPP within 16-lane rows (quad permutes,
// then half-row and row mirrors), permlane swaps across rows and halves.
__device__ __forceinline__ float wave_max_dpp(float v) {
  auto dpp = [](float x, int ctrl) -> float {
    switch (ctrl) {
      case 0xB1: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
      case 0x4E: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
      case 0x141: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));
      default: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));
    }
  };
  v = fmaxf(v, dpp(v, 0xB1));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp(v, 0x4E));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp(v, 0x141));  // row_half_mirror: the other quad of the half-row
  v = fmaxf(v, dpp(v, 0x140));  // row_mirror: the other half of the row
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));  // rows 0+1, 2+3
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));  // both halves
}

// Mask and lists from the block energies (selection.py:183-195 and
// kernel.py:141-184) in 32-bit arithmetic (the host routes geometries whose
// key positions need more bits elsewhere).  Wave w compacts the blocks
// [w * span, (w + 1) * span) 64 at a time with ballots: one pass counts, the
// waves' counts are exchanged through LDS, a second pass writes each block's
// positions (selected ascending, then the rest ascending; likewise pruned).
__device__ __forceinline__ void finish_lists(const SelectArgs& a, int h, int t, int tile_first, int tile_last,
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

// ---------------------------------------------------------------------------
// Owner path: the hook's path for D = 256 (the streaming path below keeps a
// unit's Q in registers, which D = 256 leaves no room for).  The tile's packed rows are staged in LDS once
// per 128-row pass; wave w owns the 32-block chunks c = w, w + 4, ... and, for
// each, multiplies all row groups of the pass with the chunk's pooled keys,
// which it loads straight from L2 into registers one of its chunks ahead.  A
// block's energy is summed entirely by its owner wave against the wave's lazy
// reference m_w, so no partials are merged across waves; before the
// selection every wave rescales its blocks by 2^(m_w - G), G = max m_w.
// LDS: Q pass [128][D + 8] (padded rows: conflict-free 16-byte column
// reads), E_b[Nb], wave references [4], row positions [128], scratch.
// ---------------------------------------------------------------------------
template <int D>
constexpr size_t own_lds_bytes(int64_t Nb) {
  return static_cast<size_t>(kRowsPerPass) * (D + 8) * 2 + kRowsPerPass * 8 + static_cast<size_t>(Nb) * 4 +
         4 * 4 + kRowsPerPass * 4 + 16 * 4;
}

// A row group's 16 scores per lane sum to at most 16 * 2^kWaveSlack while no
// score exceeds the wave reference by more than kWaveSlack; a sum above
// kRaiseSum therefore means some score exceeds it by more than kWaveSlack - 4,
// and the reference is raised to the wave's largest score before the sum is
// taken again.
constexpr float kRaiseSum = 65536.f;  // 2^kWaveSlack
static_assert(kWaveSlack == 16.f, "kRaiseSum is 2^kWaveSlack");

template <typename T, int D>
__global__ __launch_bounds__(kThreads, 2) __attribute__((amdgpu_waves_per_eu(1, 2))) void select_own_kernel(SelectArgs a) {
  constexpr int KS = D / 16;  // MFMA k-steps over the head dimension
  constexpr int LDQ = D + 8;
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* qs = reinterpret_cast<uint16_t*>(smem);
  int64_t* qoff = reinterpret_cast<int64_t*>(smem + static_cast<size_t>(kRowsPerPass) * LDQ * 2);  // row -> q element, -1: zeros
  float* eb = reinterpret_cast<float*>(qoff + kRowsPerPass);
  float* xm = eb + a.Nb;  // [4] wave references
  int* rpos = reinterpret_cast<int*>(xm + 4);  // local query position, -1: no such row
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

  // K-bar fragment k of a chunk: the lane's block row c*32 + l32, data chunk
  // 2k + hf (16 bytes, immediate offset 32 k); blocks past nfv read zeros
  const rsrc_t pkr = make_rsrc(static_cast<const uint16_t*>(a.pk) + ti.h * a.pk_hs,
                               static_cast<uint32_t>(a.Nb * D * 2));
  auto load_kbar = [&](int c, u32x4 (&kf)[KS]) {
    const int b = c * 32 + l32;
    const uint32_t base = (c < nchunks && b < nfv) ? static_cast<uint32_t>((b * D + hf * 8) * 2) : kOOB;
#pragma unroll
    for (int k = 0; k < KS; ++k) kf[k] = buf_load16(pkr, base + k * 32);
  };
  // S = Q . Kbar^T for row group rg of the pass: a lane holds rows
  // (j/4)*8 + hf*4 + j%4 of the group, block c*32 + l32
  const uint16_t* qrow = qs + l32 * LDQ + hf * 8;
  auto load_q = [&](int rg, u32x4 (&qf)[KS]) {
#pragma unroll
    for (int k = 0; k < KS; ++k) qf[k] = load16(qrow + rg * 32 * LDQ + k * 16);
  };
  auto mma = [&](const u32x4 (&qf)[KS], const u32x4 (&kf)[KS]) {
    f32x16 acc = {};
#pragma unroll
    for (int k = 0; k < KS; ++k) acc = Elem<T>::mfma32(as_vec8<T>(qf[k]), as_vec8<T>(kf[k]), acc);
    return acc;
  };
  auto qk = [&](int rg, const u32x4 (&kf)[KS]) {
    u32x4 qf[KS];
    load_q(rg, qf);
    return mma(qf, kf);
  };
  // the same by inline-asm reads: fragment k of group RG at a fixed offset
  // from the lane's row of group 0
  constexpr bool kResident = D <= 128;  // Q of the pass held in registers
  const uint32_t qaddr = lds_addr(qrow);
  auto read_q = [&](auto rgc, u32x4 (&qf)[KS]) {
    constexpr int rg = decltype(rgc)::value;
    StaticFor<0, KS>::run([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      qf[k] = lds_read_b128<true, (rg * 32 * LDQ + k * 16) * 2>(qaddr);
    });
  };
  auto mma_wait = [&](u32x4 (&qf)[KS], const u32x4 (&kf)[KS]) {
    f32x16 acc = {};
    StaticFor<0, KS>::run([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      constexpr int younger = KS - 1 - k < 15 ? KS - 1 - k : 15;
      lgkm_wait<true, younger>(qf[k]);
      acc = Elem<T>::mfma32(as_vec8<T>(qf[k]), as_vec8<T>(kf[k]), acc);
    });
    return acc;
  };

  float mref = neg_inf();  // wave reference m_w (log2 units, wave-uniform)
  // sum over the lane's 16 scores of 2^(s sc2 - m_w), those with ok(j)
  auto exp_sum = [&](const f32x16& s, auto ok) {
    const float bias = -mref;
    float e0 = ok(0) ? exp2_fast(fmaf(s[0], sc2, bias)) : 0.f;
    float e1 = ok(1) ? exp2_fast(fmaf(s[1], sc2, bias)) : 0.f;
#pragma unroll
    for (int j = 2; j < 16; j += 2) {
      e0 += ok(j) ? exp2_fast(fmaf(s[j], sc2, bias)) : 0.f;
      e1 += ok(j + 1) ? exp2_fast(fmaf(s[j + 1], sc2, bias)) : 0.f;
    }
    return e0 + e1;
  };
  // raise m_w to the wave's largest score among those with ok(j): rescale
  // the chunk's running sum and every energy this wave has stored (rare)
  auto raise = [&](const f32x16& s, auto ok, float& eacc) {
    float lm = neg_inf();
#pragma unroll
    for (int j = 0; j < 16; ++j) lm = ok(j) ? fmaxf(lm, s[j]) : lm;
    const float m_new = wave_max_any(lm) * sc2;
    const float f = (mref == neg_inf()) ? 0.f : exp2_fast(mref - m_new);
    eacc *= f;
    for (int cc = wave; cc < nchunks; cc += 4) {
      const int bb = cc * 32 + l32;
      if (hf == 0 && bb < nfv) eb[bb] *= f;
    }
    mref = m_new;
  };

  for (int64_t rc = 0; rc < R; rc += kRowsPerPass) {
    __syncthreads();  // the previous pass is done with qs, qoff and rpos
    if (tid < kRowsPerPass) {
      const int64_t pr = rc + tid;
      int p = -1;
      int64_t off = -1;
      if (pr < R) {
        const int64_t gg = pr / a.tq;
        p = static_cast<int>(ti.t * a.tq + (pr - gg * a.tq));
        if (p < a.Lq) off = (ti.h * a.G + gg) * a.q_hs + static_cast<int64_t>(p) * a.q_rs;
      }
      rpos[tid] = p;
      qoff[tid] = off;
    }
    __syncthreads();
    // Stage 128 packed rows of Q (zeros past the tile or the valid length),
    // every load issued before the stores.
    {
      constexpr int QN = kRowsPerPass * (D / 8) / kThreads;
      static_assert(kRowsPerPass * (D / 8) % kThreads == 0, "Q staging splits evenly");
      u32x4 qst[QN];
#pragma unroll
      for (int i = 0; i < QN; ++i) {
        const int e = tid + i * kThreads;
        const int r = e / (D / 8);
        const int64_t off = qoff[r];
        qst[i] = off >= 0 ? load16(static_cast<const uint16_t*>(a.q) + off + (e - r * (D / 8)) * 8)
                          : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int i = 0; i < QN; ++i) {
        const int e = tid + i * kThreads;
        const int r = e / (D / 8);
        store16(qs + r * LDQ + (e - r * (D / 8)) * 8, qst[i]);
      }
    }
    __syncthreads();
    const int64_t rows_here = (R - rc) < kRowsPerPass ? (R - rc) : kRowsPerPass;
    const int nrg = static_cast<int>((rows_here + 31) / 32);
    // per row group (wave-uniform): lowest position, and whether every row
    // is present and inside the valid length
    int rg_lo[4];
    bool rg_full[4];
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      int lo = rg < nrg ? rpos[rg * 32 + l32] : -1;
      int hi = lo;
#pragma unroll
      for (int o = 16; o >= 1; o >>= 1) {
        lo = min(lo, __shfl_xor(lo, o));
        hi = max(hi, __shfl_xor(hi, o));
      }
      rg_lo[rg] = __builtin_amdgcn_readfirstlane(lo);
      rg_full[rg] = __builtin_amdgcn_readfirstlane(static_cast<int>(lo >= 0 && hi < lq)) != 0;
    }

    bool all_full = nrg == 4;
    int min_lo = rg_lo[0];
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      all_full = all_full && rg_full[rg];
      min_lo = min(min_lo, rg_lo[rg]);
    }
    // add the chunk's energies (both halves of the wave) to E_b
    auto store_chunk = [&](int b, bool b_scored, float eacc) {
      const auto es = __builtin_amdgcn_permlane32_swap(__float_as_uint(eacc), __float_as_uint(eacc), false, false);
      const float etot = __uint_as_float(es[0]) + __uint_as_float(es[1]);
      if (hf == 0 && b_scored) eb[b] += etot;
    };
    // Q fragments of the pass: for D <= 128 every wave keeps all four row
    // groups in registers (4 x KS x 16 bytes per lane), so the MFMAs read no
    // LDS; for D = 256 they are read per row group by inline asm (reads
    // complete in order; each MFMA waits for its own fragment only).
    u32x4 qr[kResident ? 4 : 1][KS];
    if constexpr (kResident) {
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) load_q(rg, qr[rg]);
    }
    auto rg_scores = [&](auto rgc, const u32x4 (&kf)[KS]) {
      constexpr int rg = decltype(rgc)::value;
      if constexpr (kResident) {
        return mma(qr[rg], kf);
      } else {
        u32x4 qf[KS];
        read_q(rgc, qf);
        return mma_wait(qf, kf);
      }
    };
    // Fast chunk: every row of the pass sees every scored block.  With
    // resident Q the MFMAs of row group rg + 1 are interleaved with the sums
    // of group rg.
    auto chunk_fast = [&](int c, const u32x4 (&kf)[KS]) {
      const int b = c * 32 + l32;
      const bool b_scored = b < nfv;
      auto ok = [&](int) { return b_scored; };
      float eacc = 0.f;
      f32x16 acc0 = rg_scores(std::integral_constant<int, 0>{}, kf), acc1;
      StaticFor<0, 4>::run([&](auto rgc) {
        constexpr int rg = decltype(rgc)::value;
        f32x16& cur = (rg & 1) ? acc1 : acc0;
        f32x16& nxt = (rg & 1) ? acc0 : acc1;
        if constexpr (rg + 1 < 4 && kResident) nxt = rg_scores(std::integral_constant<int, rg + 1>{}, kf);
        float e = exp_sum(cur, ok);
        if constexpr (rg + 1 < 4 && kResident) {
#pragma unroll
          for (int k = 0; k < KS; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 48 / KS, 0);
          }
        }
        if (__ballot(e > kRaiseSum) != 0ull) {
          raise(cur, ok, eacc);
          e = exp_sum(cur, ok);
        }
        eacc += e;
        if constexpr (rg + 1 < 4 && !kResident) nxt = rg_scores(std::integral_constant<int, rg + 1>{}, kf);
      });
      store_chunk(b, b_scored, eacc);
    };
    // General chunk: partial passes, rows past the valid length, and blocks
    // that start after some row of the pass.
    auto chunk_gen = [&](int c, const u32x4 (&kf)[KS]) {
      const int b = c * 32 + l32;
      const bool b_scored = b < nfv;
      const int lo = max(0, b * bk - offset);
      float eacc = 0.f;
      StaticFor<0, 4>::run([&](auto rgc) {
        constexpr int rg = decltype(rgc)::value;
        if (rg < nrg) {
          const f32x16 s = rg_scores(rgc, kf);
          bool okr[16];
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int pos = rpos[rg * 32 + (j >> 2) * 8 + hf * 4 + (j & 3)];
            okr[j] = b_scored && pos >= lo && pos < lq;
          }
          auto ok = [&](int j) { return okr[j]; };
          float e = exp_sum(s, ok);
          if (__ballot(e > kRaiseSum) != 0ull) {
            raise(s, ok, eacc);
            e = exp_sum(s, ok);
          }
          eacc += e;
        }
      });
      store_chunk(b, b_scored, eacc);
    };
    auto chunk = [&](int c, const u32x4 (&kf)[KS]) {
      // lowest position that sees every scored block of the chunk
      const int lo_last = max(0, min(c * 32 + 31, nfv - 1) * bk - offset);
      if (all_full && min_lo >= lo_last) chunk_fast(c, kf);
      else chunk_gen(c, kf);
    };
    // this wave's chunks c = wave + 4 i
    for (int c = wave; c < nchunks; c += 4) {
      u32x4 kf[KS];
      load_kbar(c, kf);
      chunk(c, kf);
    }
  }
  // common reference: every wave rescales the blocks it owns by 2^(m_w - G)
  if (lane == 0) xm[wave] = mref;
  __syncthreads();
  const float g = fmaxf(fmaxf(xm[0], xm[1]), fmaxf(xm[2], xm[3]));
  const float f = (mref == neg_inf()) ? 0.f : exp2_fast(mref - g);
  for (int cc = wave; cc < nchunks; cc += 4) {
    const int bb = cc * 32 + l32;
    if (hf == 0 && bb < nfv) eb[bb] *= f;
  }
  __syncthreads();
  finish_lists(a, static_cast<int>(ti.h), static_cast<int>(ti.t), static_cast<int>(ti.tile_first),
              static_cast<int>(ti.tile_last), nfv, eb, fred, ired);
}

// ---------------------------------------------------------------------------
// Streaming path: the hook's path as a persistent kernel.  Each workgroup
// walks the tiles bid, bid + grid, ... (latest tiles first) in units of
// StreamGeom::ROWS packed query rows.  A unit's rows are filled into the
// LDS slot by asynchronous buffer loads (rows padded by one 16-byte
// granule: conflict-free fragment reads) and copied into registers by every
// wave, so the MFMAs read registers only.  Wave w owns the 32-block chunks
// c = w, w + 4, ... of the tile; while the chunks run, the slot holds one
// pooled-key chunk per wave, filled one chunk ahead (pooled keys are re-read
// for every tile and the query stream evicts them from L2).  The next
// unit's Q fill is issued after the chunk loop and lands during the tile's
// finish, which compacts only the blocks that start inside the causal
// range (the lists past it are the identity).
// ---------------------------------------------------------------------------
template <int D, bool SWZ>
struct StreamGeom {
  static constexpr int KS = D / 16;
  static constexpr int NRG = D <= 128 ? 4 : 2;  // 32-row groups per unit (Q registers: NRG x KS x 16 B)
  static constexpr int ROWS = NRG * 32;
  // pooled-key chunk rows: KROWB bytes (a power of two), 16-byte granule g of
  // row r stored at granule g ^ kswz(r) (conflict-free fragment reads)
  static constexpr int KROWB = D * 2 <= 128 ? 128 : 256;
  static constexpr int KG = KROWB / 16;     // granules per row
  static constexpr int RPI = 1024 / KROWB;  // rows per fill instruction
  static_assert(!SWZ || D * 2 == KROWB, "swizzled Q rows are exactly one power-of-two row");
  // Q rows in the slot: SWZ, the pooled-key layout (the host checks that a
  // fill instruction's rows share one query head and 32-bit row offsets);
  // otherwise padded by one granule
  static constexpr int QROWB = SWZ ? KROWB : (D / 8 + 1) * 16;
  static constexpr int RC = QROWB / 16;     // granules per Q row
  static constexpr int NF = (ROWS * RC + 4 * 64 - 1) / (4 * 64);  // Q fill instructions per wave
  static constexpr int SLOT = NF * 4 * 1024 > 4 * 32 * KROWB ? NF * 4 * 1024 : 4 * 32 * KROWB;
  // registers for the next row group's scores while the sums of one run
  // (Q NRG x KS x 4 + pooled keys KS x 4 + two accumulators of 16)
  static constexpr bool PIPE = NRG * KS * 4 + KS * 4 + 32 <= 160;
  // one pooled-key chunk per wave in the Q slot, which is idle while the
  // chunks run
  static constexpr int KSLOT = 32 * KROWB;
  static constexpr int NFK = KSLOT / 1024;  // fill instructions per chunk
  static_assert(4 * KSLOT <= SLOT, "four pooled-key slots fit in the Q slot");
  static __device__ __forceinline__ int kswz(int row) { return KG == 16 ? (row & 15) : ((row >> 1) & 7); }
  // kswz(RPI j + lr) = swz_inst(j) ^ swz_lane(lr) for lr < RPI (disjoint bits)
  static constexpr int swz_inst(int j) { return KG == 16 ? 4 * (j & 3) : 4 * (j & 1); }
  static __device__ __forceinline__ uint32_t swz_lane(uint32_t lr) { return KG == 16 ? lr : (lr >> 1); }
};

// dynamic LDS (the Q slot is a separate static array, so that the
// compiler's wait for the asynchronous fills covers reads of the slot only):
// E_b[Nb], row positions [256], wave references [4], wave maxima [4],
// list counts [8]
constexpr size_t stream_lds_bytes(int64_t Nb) { return static_cast<size_t>(Nb) * 4 + (256 + 4 + 4 + 8) * 4; }

template <typename T, int D, bool SWZ>
__global__ __launch_bounds__(kThreads, 2) __attribute__((amdgpu_waves_per_eu(1, 2))) void select_stream_kernel(
    SelectArgs a) {
  using SG = StreamGeom<D, SWZ>;
  constexpr int KS = SG::KS;
  constexpr int NRG = SG::NRG;
  constexpr int ROWS = SG::ROWS;
  constexpr int RC = SG::RC;
  __shared__ __align__(1024) unsigned char qslot[SG::SLOT];
  extern __shared__ __align__(16) unsigned char smem[];
  const int Nb = static_cast<int>(a.Nb);
  float* eb = reinterpret_cast<float*>(smem);      // block energies against the owner's m_w
  int* rpos = reinterpret_cast<int*>(eb + Nb);     // [ROWS] unit row -> position, -1: no such row
  float* xm = reinterpret_cast<float*>(rpos + 256);  // [4] wave references m_w
  float* wmx = xm + 4;                             // [4] wave maxima of E_b
  int* ired = reinterpret_cast<int*>(wmx + 4);     // [8] list counts

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hf = lane >> 5;
  const int Hkv = static_cast<int>(a.Hkv);
  const int Nt = static_cast<int>(a.Nt);
  const int tq = static_cast<int>(a.tq);
  const int R = static_cast<int>(a.G * a.tq);
  const int npass = (R + ROWS - 1) / ROWS;
  const int lq = static_cast<int>(a.Lq);
  const int offset = static_cast<int>(a.offset);
  const int bk = static_cast<int>(a.bk);
  const float sc2 = a.scale * kLog2e;  // > 0 on this path
  const int total = Hkv * Nt;
  const uint32_t tq_magic = a.tq_magic;
  // pr / tq for pr * tq < 2^32 (host-checked): multiply by ceil(2^32 / tq)
  auto div_tq = [&](int pr) { return static_cast<int>(__umulhi(static_cast<uint32_t>(pr), tq_magic)); };

  // ---- fills: fill instruction i of this wave writes LDS granules
  // [64 (4 i + wave), 64 (4 i + wave + 1)) of the slot; granule p holds row
  // p / RC, data granule p % RC (the last granule of a row is padding) ----
  // Arguments used once per tile are read again from the argument segment
  // (scalar cache) through a pointer the compiler cannot hoist: kept in
  // registers across the persistent loop they would exhaust the SGPRs.
  typedef __attribute__((address_space(4))) const SelectArgs* kernarg_args;
  auto fresh = [&]() {
    // the kernel's only argument sits at the start of its argument segment
    kernarg_args p = (kernarg_args)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return p;
  };
  // Workgroup barrier that leaves the asynchronous Q fill in flight: only
  // this kernel's LDS writes (ds_*) must be visible across it, and nothing
  // reads the Q slot before the next vm_wait<0> + __syncthreads.  (A plain
  // __syncthreads would also wait for the fill.)
  auto barrier_lds = []() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
  auto issue_fill = [&](int tile_i, int pass) {
    typedef __attribute__((address_space(3))) void* lds_ptr;
    kernarg_args f = fresh();
    const int h = tile_i % Hkv;
    const int t = Nt - 1 - tile_i / Hkv;
    const uint32_t q_hs = static_cast<uint32_t>(f->q_hs), q_rs = static_cast<uint32_t>(f->q_rs);
    const uint32_t q_bytes = static_cast<uint32_t>(((f->G - 1) * f->q_hs + (f->Lq - 1) * f->q_rs + D) * 2);
    const rsrc_t qr = make_rsrc(static_cast<const uint16_t*>(f->q) + h * f->G * f->q_hs, q_bytes);
    // recomputed per call rather than kept live through the chunk loop
    uint32_t ln = static_cast<uint32_t>(lane);
    asm volatile("" : "+v"(ln));
    if constexpr (SWZ) {
      // instruction j = 4 i + wave fills rows RPI j + lr (lr = lane / KG), all
      // of one query head: scalar row offsets, granule (lane % KG) ^ kswz
      const uint32_t lr = ln / SG::KG;
      const uint32_t lanepart = lr * q_rs * 2u + 16u * ((ln % SG::KG) ^ SG::swz_lane(lr));
#pragma unroll
      for (int i = 0; i < SG::NF; ++i) {
        const int j = i * 4 + wave;
        const int pr0 = pass * ROWS + j * SG::RPI;
        const int g = div_tq(pr0);
        const int pos0 = t * tq + pr0 - g * tq;
        const uint32_t sbase = (static_cast<uint32_t>(g) * q_hs + static_cast<uint32_t>(pos0) * q_rs) * 2u;
        // the scalar offset stays uniform (sbase < 2^31): an invalid lane's
        // kOOB + sbase is still past the range and reads zeros
        const bool ok = (j * SG::RPI < ROWS) & (pr0 < R) & (static_cast<int>(lr) < lq - pos0);
        const uint32_t voff = ok ? (lanepart ^ (16u * SG::swz_inst(j))) : kOOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(qr, (lds_ptr)(qslot + j * 1024), 16, voff, sbase, 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < SG::NF; ++i) {
        const int p = (i * 4 + wave) * 64 + static_cast<int>(ln);
        const int row = p / RC;
        const int gr = p - row * RC;
        const int pr = pass * ROWS + row;
        const int g = div_tq(pr);
        const int pos = t * tq + pr - g * tq;
        const bool ok = (row < ROWS) & (gr < D / 8) & (pr < R) & (pos < lq);
        const uint32_t off = ok ? (g * q_hs + pos * q_rs + gr * 8) * 2 : kOOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(qr, (lds_ptr)(qslot + (i * 4 + wave) * 1024), 16, off, 0, 0, 0);
      }
    }
  };

  // Pooled keys of chunk c into this wave's slot: fill instruction i, lane
  // -> slot granule p = 64 i + lane, row p / KG, holding data granule
  // (p % KG) ^ kswz(row) of block c*32 + row.  Blocks past nfv may hold any
  // in-range data (their scores are masked); padding granules of D = 96
  // and blocks past Nb load zeros.
  unsigned char* const kslot = qslot + wave * SG::KSLOT;
  auto fill_kbar = [&](const rsrc_t& pkr, int c) {
    typedef __attribute__((address_space(3))) void* lds_ptr;
    uint32_t ln = static_cast<uint32_t>(lane);  // recomputed per call rather than kept live
    asm volatile("" : "+v"(ln));
    const uint32_t cbase = static_cast<uint32_t>(c) * 32u * D * 2u;
    if constexpr (SWZ) {
      // instruction i fills rows RPI i + lr (lr = lane / KG): byte
      // (RPI i + lr) KROWB + 16 ((lane % KG) ^ kswz(row)) of the chunk
      const uint32_t lr = ln / SG::KG;
      const uint32_t lanepart = lr * SG::KROWB + 16u * ((ln % SG::KG) ^ SG::swz_lane(lr));
#pragma unroll
      for (int i = 0; i < SG::NFK; ++i) {
        const uint32_t voff = lanepart ^ (16u * SG::swz_inst(i));
        const uint32_t soff = cbase + i * 1024u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(pkr, (lds_ptr)(kslot + i * 1024), 16, voff, soff, 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < SG::NFK; ++i) {
        const uint32_t row = (i * 64u + ln) / SG::KG;
        const uint32_t gr = ((i * 64u + ln) % SG::KG) ^ static_cast<uint32_t>(SG::kswz(static_cast<int>(row)));
        const uint32_t off = gr < D / 8 ? cbase + (row * D + gr * 8u) * 2u : kOOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(pkr, (lds_ptr)(kslot + i * 1024), 16, off, 0, 0, 0);
      }
    }
  };
  // fragment k of the chunk in the slot: block row l32, data granule
  // 2k + hf, i.e. byte (2k + hf) ^ kswz(l32) of the row: the k-dependent
  // part is an XOR of 32 k on a row-aligned base
  const uint32_t kread = lds_addr(kslot) + l32 * SG::KROWB + ((16 * hf) ^ (16 * SG::kswz(l32)));
  auto read_kbar = [&](u32x4 (&kf)[KS]) {
    typedef __attribute__((address_space(3))) const u32x4* lds_u32x4p;
#pragma unroll
    for (int k = 0; k < KS; ++k) kf[k] = *(lds_u32x4p)(static_cast<uintptr_t>(kread ^ (32 * k)));
  };
  auto mma = [&](const u32x4 (&qf)[KS], const u32x4 (&kf)[KS]) {
    f32x16 acc = {};
#pragma unroll
    for (int k = 0; k < KS; ++k) acc = Elem<T>::mfma32(as_vec8<T>(qf[k]), as_vec8<T>(kf[k]), acc);
    return acc;
  };

  float mref = neg_inf();  // wave reference m_w (log2 units, wave-uniform)
  // sum over the lane's 16 scores of 2^(s sc2 - m_w), those with ok(j)
  auto exp_sum = [&](const f32x16& s, auto ok) {
    const float bias = -mref;
    float e0 = ok(0) ? exp2_fast(fmaf(s[0], sc2, bias)) : 0.f;
    float e1 = ok(1) ? exp2_fast(fmaf(s[1], sc2, bias)) : 0.f;
#pragma unroll
    for (int j = 2; j < 16; j += 2) {
      e0 += ok(j) ? exp2_fast(fmaf(s[j], sc2, bias)) : 0.f;
      e1 += ok(j + 1) ? exp2_fast(fmaf(s[j + 1], sc2, bias)) : 0.f;
    }
    return e0 + e1;
  };

  if (static_cast<int>(blockIdx.x) >= total) return;
  issue_fill(blockIdx.x, 0);
  for (int tile_i = blockIdx.x; tile_i < total; tile_i += gridDim.x) {
    const int h = tile_i % Hkv;
    const int t = Nt - 1 - tile_i / Hkv;  // latest tiles (longest rows) first
    const int tile_first = offset + t * tq;
    const int tile_last = min(tile_first + tq, offset + lq) - 1;
    const int nfv = min(Nb, max(0, (tile_last + 1) / bk));  // blocks that end inside the causal range
    const int nchunks = (nfv + 31) / 32;
    kernarg_args ta = fresh();
    const rsrc_t pkr = make_rsrc(static_cast<const uint16_t*>(ta->pk) + static_cast<int64_t>(h) * ta->pk_hs,
                                 static_cast<uint32_t>(Nb * D * 2));
    mref = neg_inf();
    float emax_w = 0.f;  // largest E_b of this wave's blocks (last pass)

    for (int pass = 0; pass < npass; ++pass) {
      vm_wait<0>();
      __syncthreads();  // the unit's fill has landed; the previous unit and finish are done with LDS
      if (tid < ROWS) {
        const int pr = pass * ROWS + tid;
        rpos[tid] = pr < R ? t * tq + pr - div_tq(pr) * tq : -1;
      }
      // the unit's Q fragments: row rg*32 + l32, data granules 2k + hf
      u32x4 qr[NRG][KS];
      if constexpr (SWZ) {
        // kswz(rg*32 + l32) = kswz(l32): the same XOR pattern as the pooled keys
        typedef __attribute__((address_space(3))) const u32x4* lds_u32x4p;
        const uint32_t qread = lds_addr(qslot) + l32 * SG::QROWB + ((16 * hf) ^ (16 * SG::kswz(l32)));
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg)
#pragma unroll
          for (int k = 0; k < KS; ++k)
            qr[rg][k] = *(lds_u32x4p)(static_cast<uintptr_t>((qread ^ (32 * k)) + rg * 32 * SG::QROWB));
      } else {
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg)
#pragma unroll
          for (int k = 0; k < KS; ++k)
            qr[rg][k] = *reinterpret_cast<const u32x4*>(qslot + ((rg * 32 + l32) * RC + 2 * k + hf) * 16);
      }
      __syncthreads();  // rpos written; every wave holds its Q, so the slot may be refilled
      // per row group (wave-uniform): lowest position, and whether every
      // row is present and inside the valid length
      const int nrg = (min(R - pass * ROWS, ROWS) + 31) / 32;
      bool all_full = nrg == NRG;
      int min_lo = 0x7fffffff;
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
        int lo = rpos[rg * 32 + l32];
        int hi = lo;
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) {
          lo = min(lo, __shfl_xor(lo, o));
          hi = max(hi, __shfl_xor(hi, o));
        }
        lo = __builtin_amdgcn_readfirstlane(lo);
        hi = __builtin_amdgcn_readfirstlane(hi);
        all_full = all_full && lo >= 0 && hi < lq;
        min_lo = min(min_lo, lo);
      }

      // raise m_w to the wave's largest score among those with ok(j):
      // rescale the running sums and every energy this wave has stored
      // (rare; entries of chunks not yet stored in the first pass are stale
      // and will be overwritten)
      auto raise = [&](const f32x16& s, auto ok, float& eacc) {
        float lm = neg_inf();
#pragma unroll
        for (int j = 0; j < 16; ++j) lm = ok(j) ? fmaxf(lm, s[j]) : lm;
        const float m_new = wave_max_dpp(lm) * sc2;
        const float f = (mref == neg_inf()) ? 0.f : exp2_fast(mref - m_new);
        eacc *= f;
        emax_w *= f;
        for (int cc = wave; cc < nchunks; cc += 4) {
          const int bb = cc * 32 + l32;
          if (hf == 0 && bb < nfv) eb[bb] *= f;
        }
        mref = m_new;
      };
      // add the chunk's energies (both halves of the wave) to E_b
      auto store_chunk = [&](int b, bool b_scored, float eacc) {
        const auto es = __builtin_amdgcn_permlane32_swap(__float_as_uint(eacc), __float_as_uint(eacc), false, false);
        float etot = __uint_as_float(es[0]) + __uint_as_float(es[1]);
        if (hf == 0 && b_scored) {
          if (pass > 0) etot += eb[b];
          eb[b] = etot;
        }
        if (pass == npass - 1 && b_scored) emax_w = fmaxf(emax_w, etot);
      };
      // this wave's chunks c = wave + 4 i: chunk c + 4 is filled into the
      // slot while chunk c runs from registers
      if (wave < nchunks) fill_kbar(pkr, wave);
      for (int c = wave; c < nchunks; c += 4) {
        u32x4 kf[KS];
        vm_wait<0>();
        read_kbar(kf);
        if (c + 4 < nchunks) {
          // the slot's reads must complete before the fill overwrites it
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          fill_kbar(pkr, c + 4);
        }
        const int b = c * 32 + l32;
        const bool b_scored = b < nfv;
        float eacc = 0.f;
        // lowest position that sees every scored block of the chunk
        const int lo_last = max(0, min(c * 32 + 31, nfv - 1) * bk - offset);
        if (all_full && min_lo >= lo_last) {
          // every row of the unit sees every scored block; the MFMAs of row
          // group rg + 1 are interleaved with the sums of group rg
          auto ok = [&](int) { return b_scored; };
          f32x16 acc0 = mma(qr[0], kf), acc1;
          StaticFor<0, NRG>::run([&](auto rgc) {
            constexpr int rg = decltype(rgc)::value;
            f32x16& cur = (rg & 1) ? acc1 : acc0;
            f32x16& nxt = (rg & 1) ? acc0 : acc1;
            if constexpr (rg + 1 < NRG && SG::PIPE) nxt = mma(qr[rg + 1], kf);
            float e = exp_sum(cur, ok);
            if constexpr (rg + 1 < NRG && SG::PIPE) {
#pragma unroll
              for (int k = 0; k < KS; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 48 / KS, 0);
              }
            }
            if (__ballot(e > kRaiseSum) != 0ull) {
              raise(cur, ok, eacc);
              e = exp_sum(cur, ok);
            }
            eacc += e;
            if constexpr (rg + 1 < NRG && !SG::PIPE) nxt = mma(qr[rg + 1], kf);
          });
        } else {
          // partial units, rows past the valid length, blocks that start
          // after some row of the unit: each score is tested
          const int lo = max(0, b * bk - offset);
          StaticFor<0, NRG>::run([&](auto rgc) {
            constexpr int rg = decltype(rgc)::value;
            if (rg < nrg) {
              const f32x16 sc = mma(qr[rg], kf);
              auto ok = [&](int j) {
                const int pos = rpos[rg * 32 + (j >> 2) * 8 + hf * 4 + (j & 3)];
                return b_scored && pos >= lo && pos < lq;
              };
              float e = exp_sum(sc, ok);
              if (__ballot(e > kRaiseSum) != 0ull) {
                raise(sc, ok, eacc);
                e = exp_sum(sc, ok);
              }
              eacc += e;
            }
          });
        }
        store_chunk(b, b_scored, eacc);
      }
      if (pass + 1 < npass) {
        __syncthreads();  // every wave is done with its pooled-key slot
        issue_fill(tile_i, pass + 1);
      }
    }

    // ---- finish (selection.py:183-195, kernel.py:141-184) ----
    const float wm = wave_max_dpp(emax_w);
    if (lane == 0) {
      xm[wave] = mref;
      wmx[wave] = wm;
    }
    __syncthreads();  // xm, wmx written; every wave is done with its pooled-key slot
    if (tile_i + static_cast<int>(gridDim.x) < total) issue_fill(tile_i + gridDim.x, 0);  // lands during the finish
    // E_b = eb[b] 2^(m_w - G) with w the owner of b and G = max m_w
    const float g = fmaxf(fmaxf(xm[0], xm[1]), fmaxf(xm[2], xm[3]));
    float fw[4], emax = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      fw[w] = (xm[w] == neg_inf()) ? 0.f : exp2_fast(xm[w] - g);
      emax = fmaxf(emax, wmx[w] * fw[w]);
    }
    kernarg_args fa = fresh();
    const float thr = fa->alpha * emax;
    const int nvis = min(Nb, tile_last / bk + 1);  // blocks that start inside the causal range
    const int sink = static_cast<int>(fa->sink);
    const int first_minus_window = tile_first - static_cast<int>(fa->window);
    const int lk = static_cast<int>(fa->Lk);
    const bool tail = t >= Nt - static_cast<int>(fa->last_n);
    // branch-free: every lane reads an E_b (clamped index; entries past
    // nfv are discarded), so no LDS read is left pending in a branch
    auto flags = [&](int b, bool& sel, bool& pru) {
      const float e_raw = eb[min(b, Nb - 1)];
      const int w = (b >> 5) & 3;
      const float f = w == 0 ? fw[0] : (w == 1 ? fw[1] : (w == 2 ? fw[2] : fw[3]));
      const float E = b < nfv ? e_raw * f : 0.f;
      const int bs = b * bk;
      const int be = bs + bk;
      const bool forced = bs < sink || be > first_minus_window || tail;
      sel = (E >= thr || forced) && bs <= tile_last;
      pru = !sel && min(be, lk) <= tile_first;
    };
    const int span = ((nvis + 4 * 64 - 1) / (4 * 64)) * 64;
    const int w0 = min(nvis, wave * span), w1 = min(nvis, w0 + span);
    // flags evaluated once: bit it of selbits / prubits is the lane's block
    // of iteration it (span <= FPV2_MAX_BLOCKS / 4: at most 32 iterations)
    static_assert(FPV2_MAX_BLOCKS <= 4 * 64 * 32, "finish flags fit 32 bits per lane");
    int ns = 0, np = 0;
    uint32_t selbits = 0, prubits = 0;
    for (int base = w0, it = 0; base < w1; base += 64, ++it) {
      const int b = base + lane;
      bool sel, pru;
      flags(b, sel, pru);
      sel = sel && b < w1;
      pru = pru && b < w1;
      selbits |= static_cast<uint32_t>(sel) << it;
      prubits |= static_cast<uint32_t>(pru) << it;
      ns += __popcll(__ballot(sel));
      np += __popcll(__ballot(pru));
    }
    if (lane == 0) {
      ired[wave] = ns;
      ired[4 + wave] = np;
    }
    barrier_lds();
    int run_s = 0, run_p = 0, tot_s = 0, tot_p = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int cs = ired[w], cp = ired[4 + w];
      run_s += w < wave ? cs : 0;
      run_p += w < wave ? cp : 0;
      tot_s += cs;
      tot_p += cp;
    }
    const int64_t row = static_cast<int64_t>(h) * Nt + t;
    typedef __attribute__((address_space(1))) int32_t g_i32;
    typedef __attribute__((address_space(1))) uint8_t g_u8;
    g_i32* ids = (g_i32*)(fa->ids + row * Nb);
    g_i32* pids = (g_i32*)(fa->pids + row * Nb);
    g_u8* selo = fa->sel_out ? (g_u8*)(fa->sel_out + row * Nb) : nullptr;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int base = w0, it = 0; base < w1; base += 64, ++it) {
      const int b = base + lane;
      const bool sel = (selbits >> it) & 1u;
      const bool pru = (prubits >> it) & 1u;
      const uint64_t ms = __ballot(sel);
      const uint64_t mp = __ballot(pru);
      if (b < w1) {
        const int ps = run_s + __popcll(ms & below);  // selected before b
        const int pp = run_p + __popcll(mp & below);
        ids[sel ? ps : tot_s + (b - ps)] = b;
        pids[pru ? pp : tot_p + (b - pp)] = b;
        if (selo) selo[b] = sel;
      }
      run_s += __popcll(ms);
      run_p += __popcll(mp);
    }
    // blocks that start past the tile: neither selected nor pruned (the
    // host routes key lengths that do not cover the queries elsewhere)
    for (int b = nvis + tid; b < Nb; b += kThreads) {
      ids[b] = b;
      pids[b] = b;
      if (selo) selo[b] = 0;
    }
    if (tid == 0) {
      ((g_i32*)fa->counts)[row] = tot_s;
      ((g_i32*)fa->pcounts)[row] = tot_p;
    }
  }
  vm_wait<0>();
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

// compute units of the current device (the streaming grid is two
// workgroups per unit)
int cu_count() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
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
  // the hook's paths keep key positions and list entries in 32 bits
  const bool small = a.Nb * a.bk <= (1LL << 30) && a.offset + a.Lq_pad <= (1LL << 30) &&
                     a.sink <= (1LL << 30) && a.window <= (1LL << 30) && a.Nt <= (1LL << 30);
  // streaming kernel: 32-bit query offsets within one KV head's rows, exact
  // 32-bit division by tq, and key lengths that cover every query
  const int64_t q_span = (a.G - 1) * a.q_hs + (a.Lq - 1) * a.q_rs + D;
  const bool stream_ok = small && a.tq >= 2 && (a.G * a.tq + 256) * a.tq < (1LL << 32) &&
                         q_span * 2 < kMaxRsrcBytes && a.Nb * D * 2 < kMaxRsrcBytes &&
                         a.Lk > a.offset + (a.Nt - 1) * a.tq && a.Hkv * a.Nt < (1LL << 31);
  if (a.scores == nullptr && a.scale > 0.f && a.ids != nullptr && stream_ok) {
    SelectArgs s = a;
    s.tq_magic = static_cast<uint32_t>(((1ull << 32) + static_cast<uint64_t>(a.tq) - 1) / static_cast<uint64_t>(a.tq));
    const int64_t tiles = a.Hkv * a.Nt;
    const dim3 sgrid(static_cast<unsigned>(tiles < 2LL * cu_count() ? tiles : 2LL * cu_count()));
    // swizzled Q rows: a fill instruction's RPI rows belong to one query
    // head (tq, R multiples of RPI) and their row offsets keep the granule
    // bits clear (q_rs * 2 a multiple of the row size)
    const int64_t rpi = 1024 / (D * 2);
    const bool swz = (D == 64 || D == 128) && a.tq % rpi == 0 && (a.q_rs * 2) % (D * 2) == 0;
    switch (D) {
      case 64:
        return swz ? launch_with_lds(select_stream_kernel<T, 64, true>, sgrid, stream_lds_bytes(a.Nb), stream, s)
                   : launch_with_lds(select_stream_kernel<T, 64, false>, sgrid, stream_lds_bytes(a.Nb), stream, s);
      case 96: return launch_with_lds(select_stream_kernel<T, 96, false>, sgrid, stream_lds_bytes(a.Nb), stream, s);
      case 128:
        return swz ? launch_with_lds(select_stream_kernel<T, 128, true>, sgrid, stream_lds_bytes(a.Nb), stream, s)
                   : launch_with_lds(select_stream_kernel<T, 128, false>, sgrid, stream_lds_bytes(a.Nb), stream, s);
      default: break;  // D = 256: the owner path below (its registers hold no resident Q)
    }
  }
  if (a.scores == nullptr && a.scale > 0.f && a.ids != nullptr && small) {
    switch (D) {
      case 64: return launch_with_lds(select_own_kernel<T, 64>, grid, own_lds_bytes<64>(a.Nb), stream, a);
      case 96: return launch_with_lds(select_own_kernel<T, 96>, grid, own_lds_bytes<96>(a.Nb), stream, a);
      case 128: return launch_with_lds(select_own_kernel<T, 128>, grid, own_lds_bytes<128>(a.Nb), stream, a);
      case 256: return launch_with_lds(select_own_kernel<T, 256>, grid, own_lds_bytes<256>(a.Nb), stream, a);

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
