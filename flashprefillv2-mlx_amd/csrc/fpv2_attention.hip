// Block-sparse FlashAttention-2 forward with pooled mean correction, gfx950.
//
// Semantics follow the fpv2_sparse_attention Metal kernel
// (fpv2/kernel.py:187-414): for each query row, an online base-2 softmax over
// the keys of the tile's selected blocks (ascending list, stop at the first
// block past the tile's last row, causal mask on the diagonal), then — with
// mean correction — over the pooled K/V rows of the tile's pruned blocks with
// a +log2(block_k) logit shift; O /= l at the end.
//
// MI355X mapping:
//   * one workgroup = one (KV head, query tile, 128-row chunk); the tile's
//     G*tile_q packed rows (row = g*tile_q + p) share the block lists, so the
//     G query heads of a KV head share every K/V load (the hook's tile is
//     128 packed rows: one chunk);
//   * 4 waves x 32 rows; Q lives in VGPRs for the whole workgroup;
//   * S^T = K . Q^T with v_mfma_f32_32x32x16_{bf16,f16}: lane l owns query
//     row l%32 and 16 of the 32 keys of each key tile, so row max/sum need a
//     single lane-pair exchange and P feeds the next MFMA without a transpose;
//   * O^T = V^T . P^T: the rescale by exp2(m_old - m_new) is lane-local;
//   * K/V sub-tiles of 64 keys are double-buffered in LDS: the next sub-tile's
//     global loads are in flight while the current one is multiplied; V is
//     transposed on its way into LDS so both MFMA operands are 8-byte/16-byte
//     LDS reads; row strides are padded against bank conflicts;
//   * grid order puts the KV head in the low bits of the workgroup id, so the
//     round-robin dispatch over the 8 XCDs keeps one head per XCD L2 (for
//     Hkv = 8), and tiles run latest (longest) first.
#include <type_traits>

#include "fpv2_common.h"

namespace fpv2 {
namespace {

constexpr int kThreads = 256;
constexpr int kRows = 128;  // packed query rows per workgroup

// gfx950 transposing LDS read (ds_read_b64_tr_b16): within each 16-lane group
// lane i receives element i%4 of the 8-byte chunks addressed by lanes
// i/4, i/4+4, i/4+8, i/4+12.
//
// Issued as inline asm on purpose: the compiler cannot tell this read from
// the asynchronous global->LDS fills of the other stage and would otherwise
// wait for those fills before the first such read of every step, which
// serialises the fill latency with most of the step's work.  The result is
// only valid after tr_wait() (s_waitcnt lgkmcnt(0)), which takes the result
// registers as operands so their uses cannot be scheduled before it.  The
// stage read here was completed by fills_done() (vmcnt(0) + barrier).
template <int OFF>
__device__ __forceinline__ u32x2 tr_read(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field is 16 bits");
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
template <int N>
__device__ __forceinline__ void tr_wait(u32x2 (&r)[N]) {
  static_assert(N == 8, "tr_wait ties a batch of 8 reads");
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]),
                 "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7]));
}
__device__ __forceinline__ uint32_t lds_addr(const uint16_t* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint16_t*)(p)));
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [0, N).
template <int I, int N>
struct StaticFor {
  template <typename F>
  static __device__ __forceinline__ void run(F&& f) {
    if constexpr (I < N) {
      f(std::integral_constant<int, I>{});
      StaticFor<I + 1, N>::run(f);
    }
  }
};

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* pk;
  const uint16_t* pv;
  const int32_t* ids;
  const int32_t* counts;
  const int32_t* pids;
  const int32_t* pcounts;
  uint16_t* out;
  int G, Hkv, Nt, Nb, Lq, out_rows, Lk, offset, bk, tq, nchunk;
  float c_scale;  // scale * log2(e)
  float shift;    // log2(block_k)
  int64_t q_hs, k_hs, v_hs, o_hs, o_rs;
  int q_rs, k_rs, v_rs;
  uint32_t q_bytes, k_bytes, v_bytes, pooled_bytes;  // descriptor ranges
};

__device__ __forceinline__ int clampi(int x, int lo, int hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

// Keys per LDS sub-tile: 64, or 32 for the 256-wide heads (registers).
template <int D> struct SubTile { static constexpr int BN = D <= 128 ? 64 : 32; };

// LDS stage layout.  A stage holds one K and one V sub-tile, row-major with
// padded rows, viewed as a linear array of 16-byte slots so that it can be
// filled by buffer_load_dwordx4 ... lds (each wave instruction writes 64
// consecutive slots, lane i -> slot base + i).  Pad slots are loaded from an
// out-of-range offset (zeros).
template <typename T, int D, bool CORR>
struct AttnTile {
  static constexpr int BN = SubTile<D>::BN;     // keys per sub-tile
  static constexpr int DG = D / 8;              // 16-byte chunks per row
  static constexpr int SK = DG + 1;             // K row: D + 8 elements (conflict-free b128 reads)
  static constexpr int SV = DG + 4;             // V row: D + 32 elements (conflict-free transpose reads)
  static constexpr int LDK = SK * 8;
  static constexpr int LDVR = SV * 8;
  static constexpr int KS = D / 16;             // QK^T k-steps
  static constexpr int DT = D / 32;             // O^T row tiles (32 dims)
  static constexpr int NTK = BN / 32;           // S^T key tiles
  static constexpr int K_INSTR = (BN * SK + 63) / 64;  // wave instructions per K sub-tile
  static constexpr int V_INSTR = (BN * SV + 63) / 64;
  static constexpr int K_ELEMS = K_INSTR * 64 * 8;     // uint16 elements
  static constexpr int V_ELEMS = V_INSTR * 64 * 8;
  static constexpr int STAGE = K_ELEMS + V_ELEMS;
  static constexpr int WAVES = kThreads / 64;
  static constexpr int KI_PER_WAVE = (K_INSTR + WAVES - 1) / WAVES;
  static constexpr int VI_PER_WAVE = (V_INSTR + WAVES - 1) / WAVES;
};

// One K/V sub-tile of the walk: `nkeys` valid rows starting at key `key0`
// (exact phase) or at pruned-list entry `li` (correction phase).
struct Step {
  int corr;   // 0: exact keys of a selected block, 1: pooled entries of pruned blocks
  int li;     // first pruned-list entry (correction)
  int key0;   // first key (exact)
  int nkeys;  // valid rows in the sub-tile
};

template <typename T, int D, bool CORR>
__global__ __launch_bounds__(kThreads, (D <= 128 ? 2 : 1)) void sparse_attn_kernel(AttnArgs a) {
  using TL = AttnTile<T, D, CORR>;
  using vec8 = typename Elem<T>::vec8;
  constexpr int BN = TL::BN;
  // Two LDS stages as separate objects, so stage reads and the asynchronous
  // fills of the other stage are known not to alias.
  __shared__ __align__(1024) uint16_t stage0[TL::STAGE];
  __shared__ __align__(1024) uint16_t stage1[TL::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int l32 = lane & 31;
  const int hf = lane >> 5;

  // ---- workgroup -> (KV head, tile, row chunk); latest tiles first ----
  const int bid = blockIdx.x;
  const int h = bid % a.Hkv;
  const int rest = bid / a.Hkv;
  const int chunk = rest % a.nchunk;
  const int t = a.Nt - 1 - rest / a.nchunk;
  const int abs_first = a.offset + t * a.tq;
  const int last_local = min((t + 1) * a.tq, a.Lq);
  const int abs_last = a.offset + last_local - 1;

  // ---- this lane's query row ----
  const int R = a.G * a.tq;
  const int prow = chunk * kRows + wave * 32 + l32;
  const bool exists = prow < R;
  int g = 0, pos = 0;
  if (exists) {
    g = prow / a.tq;
    pos = t * a.tq + (prow - g * a.tq);
  }
  const bool row_valid = exists && pos < a.Lq;
  const int qpos_abs = a.offset + pos;

  vec8 qf[TL::KS];
  {
    const rsrc_t qr = make_rsrc(a.q + static_cast<int64_t>(h) * a.G * a.q_hs, a.q_bytes);
    const uint32_t qoff =
        row_valid ? static_cast<uint32_t>((g * a.q_hs + static_cast<int64_t>(pos) * a.q_rs + hf * 8) * 2)
                  : kOOB;
    // The softmax folds the scale into one FMA per logit and needs a positive
    // factor: for scale < 0 the queries are negated instead (s*c = (-s)*(-c)).
    const uint32_t sign = a.c_scale < 0.f ? 0x80008000u : 0u;
#pragma unroll
    for (int k = 0; k < TL::KS; ++k) {
      u32x4 v = buf_load16(qr, qoff + (row_valid ? k * 32 : 0));
      v ^= sign;
      qf[k] = as_vec8<T>(v);
    }
  }
  const float c_pos = fmaxf(fabsf(a.c_scale), 1e-30f);

  // ---- block lists of (h, t), clipped as kernel.py:555-558 ----
  const int Nb = a.Nb;
  const int64_t list_row = static_cast<int64_t>(h) * a.Nt + t;
  const int32_t* ids = a.ids + list_row * Nb;
  const int32_t* pids = a.pids + list_row * Nb;
  const int sel_count = clampi(a.counts[list_row], 0, Nb);
  const int pr_count = CORR ? clampi(a.pcounts[list_row], 0, Nb) : 0;
  const int subs = (a.bk + BN - 1) / BN;

  // The walk stops at the first listed block that starts after the tile's
  // last row (kernel.py:252): find it with one ballot per 64 entries.
  int li_end = sel_count;
  for (int base = 0; base < sel_count; base += 64) {
    const int li = base + lane;
    const bool past = li < sel_count && clampi(ids[li], 0, Nb - 1) * a.bk > abs_last;
    const uint64_t m = __ballot(past);
    if (m != 0ull) {
      li_end = base + static_cast<int>(__builtin_ctzll(m));
      break;
    }
  }
  // Exact-phase sub-tiles: every sub-tile of the blocks before li_end, the
  // last block trimmed at the tile's last row; sub-tiles of other blocks that
  // start past it (only in non-ascending lists) are skipped as empty.
  int n_sel = 0;
  if (li_end > 0) {
    const int last_blk = clampi(ids[li_end - 1], 0, Nb - 1);
    n_sel = (li_end - 1) * subs + min(subs, (abs_last - last_blk * a.bk) / BN + 1);
  }
  const int n_corr = CORR ? (pr_count + BN - 1) / BN : 0;
  const int n_steps = n_sel + n_corr;

  // Block ids of the selected list are read 64 at a time into one VGPR (lane
  // = list entry) and handed out with readlane, so producing a step costs no
  // memory round trip.  The walk state (list entry, sub-tile) advances
  // incrementally.
  int ids_base = 0;
  int ids_lanes = lane < sel_count ? clampi(ids[lane], 0, Nb - 1) : 0;
  int cur_li = 0, cur_sub = 0;
  auto next_step = [&](int it) -> Step {
    Step s;
    if (it < n_sel) {
      if (cur_li - ids_base >= 64) {
        ids_base += 64;
        const int li = ids_base + lane;
        ids_lanes = li < sel_count ? clampi(ids[li], 0, Nb - 1) : 0;
      }
      const int blk = __builtin_amdgcn_readlane(ids_lanes, cur_li - ids_base);
      s.corr = 0;
      s.li = cur_li;
      s.key0 = blk * a.bk + cur_sub * BN;
      int n = min(min(a.bk - cur_sub * BN, BN), a.Lk - s.key0);
      if (s.key0 > abs_last) n = 0;
      s.nkeys = n < 0 ? 0 : n;
      if (++cur_sub == subs) {
        cur_sub = 0;
        ++cur_li;
      }
    } else {
      s.corr = 1;
      s.li = (it - n_sel) * BN;
      s.key0 = 0;
      s.nkeys = min(pr_count - s.li, BN);
    }
    return s;
  };

  // ---- global -> LDS fills (buffer_load_dwordx4 ... lds) ----
  // Per lane and per wave instruction: the slot's row and its byte offset
  // within the row pattern (kOOB for pad slots).  Constant over the walk.
  const rsrc_t kr = make_rsrc(a.k + h * a.k_hs, a.k_bytes);
  const rsrc_t vr = make_rsrc(a.v + h * a.v_hs, a.v_bytes);
  const rsrc_t pkr = make_rsrc(a.pk + static_cast<int64_t>(h) * Nb * D, a.pooled_bytes);
  const rsrc_t pvr = make_rsrc(a.pv + static_cast<int64_t>(h) * Nb * D, a.pooled_bytes);
  // Per lane and wave instruction, the byte offset of the slot within a
  // sub-tile of consecutive rows (-1 for pad slots); rows are recomputed only
  // on the rare partial and correction sub-tiles.
  int k_pre[TL::KI_PER_WAVE], v_pre[TL::VI_PER_WAVE];
#pragma unroll
  for (int i = 0; i < TL::KI_PER_WAVE; ++i) {
    const int slot = (wave + i * TL::WAVES) * 64 + lane;
    const int r = slot / TL::SK, c = slot - r * TL::SK;
    k_pre[i] = (c < TL::DG && r < BN) ? (r * a.k_rs + c * 8) * 2 : -1;
  }
#pragma unroll
  for (int i = 0; i < TL::VI_PER_WAVE; ++i) {
    const int slot = (wave + i * TL::WAVES) * 64 + lane;
    const int r = slot / TL::SV, c = slot - r * TL::SV;
    v_pre[i] = (c < TL::DG && r < BN) ? (r * a.v_rs + c * 8) * 2 : -1;
  }

  // One K/V fill of `stage` for step s.  `rows_of` gives the slot's row
  // (BN for pad slots) and its 16-byte chunk.
  auto slot_of = [&](int j, int per_row, int& row, int& chunk) {
    const int slot = j * 64 + lane;
    row = slot / per_row;
    chunk = slot - row * per_row;
    if (chunk >= TL::DG || row >= BN) row = BN;
  };
  auto fill_step = [&](const Step& s, uint16_t* stage) {
    typedef __attribute__((address_space(3))) void* lds_ptr;
    if (!s.corr && s.nkeys == BN) {  // full exact sub-tile: offsets only
      const int kbase = s.key0 * a.k_rs * 2;
      const int vbase = s.key0 * a.v_rs * 2;
#pragma unroll
      for (int i = 0; i < TL::KI_PER_WAVE; ++i) {
        const int j = wave + i * TL::WAVES;
        if (j < TL::K_INSTR) {
          const uint32_t off = k_pre[i] >= 0 ? static_cast<uint32_t>(kbase + k_pre[i]) : kOOB;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (lds_ptr)(stage + j * 512), 16, off, 0, 0, 0);
        }
      }
#pragma unroll
      for (int i = 0; i < TL::VI_PER_WAVE; ++i) {
        const int j = wave + i * TL::WAVES;
        if (j < TL::V_INSTR) {
          const uint32_t off = v_pre[i] >= 0 ? static_cast<uint32_t>(vbase + v_pre[i]) : kOOB;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (lds_ptr)(stage + TL::K_ELEMS + j * 512), 16,
                                                   off, 0, 0, 0);
        }
      }
    } else if (!s.corr) {  // partial exact sub-tile (end of the keys / of the block)
      const int kbase = s.key0 * a.k_rs * 2;
      const int vbase = s.key0 * a.v_rs * 2;
#pragma unroll
      for (int i = 0; i < TL::KI_PER_WAVE; ++i) {
        const int j = wave + i * TL::WAVES;
        if (j < TL::K_INSTR) {
          int row, chunk;
          slot_of(j, TL::SK, row, chunk);
          const uint32_t off = row < s.nkeys ? static_cast<uint32_t>(kbase + k_pre[i]) : kOOB;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (lds_ptr)(stage + j * 512), 16, off, 0, 0, 0);
        }
      }
#pragma unroll
      for (int i = 0; i < TL::VI_PER_WAVE; ++i) {
        const int j = wave + i * TL::WAVES;
        if (j < TL::V_INSTR) {
          int row, chunk;
          slot_of(j, TL::SV, row, chunk);
          const uint32_t off = row < s.nkeys ? static_cast<uint32_t>(vbase + v_pre[i]) : kOOB;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (lds_ptr)(stage + TL::K_ELEMS + j * 512), 16,
                                                   off, 0, 0, 0);
        }
      }
    } else {  // correction: gather pooled rows of the pruned blocks
#pragma unroll
      for (int i = 0; i < TL::KI_PER_WAVE; ++i) {
        const int j = wave + i * TL::WAVES;
        if (j < TL::K_INSTR) {
          int row, chunk;
          slot_of(j, TL::SK, row, chunk);
          const bool ok = row < s.nkeys;
          const int blk = clampi(pids[ok ? s.li + row : s.li], 0, Nb - 1);
          const uint32_t off = ok ? static_cast<uint32_t>((blk * D + chunk * 8) * 2) : kOOB;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(pkr, (lds_ptr)(stage + j * 512), 16, off, 0, 0, 0);
        }
      }
#pragma unroll
      for (int i = 0; i < TL::VI_PER_WAVE; ++i) {
        const int j = wave + i * TL::WAVES;
        if (j < TL::V_INSTR) {
          int row, chunk;
          slot_of(j, TL::SV, row, chunk);
          const bool ok = row < s.nkeys;
          const int blk = clampi(pids[ok ? s.li + row : s.li], 0, Nb - 1);
          const uint32_t off = ok ? static_cast<uint32_t>((blk * D + chunk * 8) * 2) : kOOB;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(pvr, (lds_ptr)(stage + TL::K_ELEMS + j * 512), 16,
                                                   off, 0, 0, 0);
        }
      }
    }
  };
  // Wait for this wave's outstanding fills (vmcnt = 0), then for all waves.
  auto fills_done = [&]() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0) expcnt(7) lgkmcnt(15)
    __syncthreads();
  };

  // ---- accumulators ----
  // Online softmax in log2 units with a lazily updated reference max m_ref:
  // P = exp2(s*c + shift - m_ref) may exceed 1 by up to 2^kRescaleSlack, and
  // O / l are rescaled only when some row's max grows past that, so the
  // common case costs no rescale at all.  The result O / l is unchanged.
  constexpr float kRescaleSlack = 8.0f;
  f32x16 o[TL::DT];
#pragma unroll
  for (int i = 0; i < TL::DT; ++i) o[i] = f32x16{};
  float m_ref = neg_inf();
  float l_run = 0.f;

  // Per-lane pieces of the transpose-read address of V^T fragments: lane j of
  // a 16-lane group reads row (j/4) and columns 4*(j%4).. of a 4-key x 16-dim
  // patch; the transpose hands lane i the 4 keys of dim d0 + i.
  const int tr_row = (lane & 15) >> 2;
  const int tr_col = (lane & 3) * 4 + ((lane >> 4) & 1) * 16;

  // One 32-key slice (key tile kt of the sub-tile): S^T, mask, online softmax
  // update, P, then O^T += V^T . P^T.  Slicing the 64-key sub-tile keeps only
  // 16 S and 8 P registers live.
  auto compute_slice = [&](const Step& s, const uint16_t* stage, int kt) {
    const uint16_t* ks = stage;
    const uint16_t* vs = stage + TL::K_ELEMS;
    f32x16 st = f32x16{};
#pragma unroll
    for (int k = 0; k < TL::KS; ++k) {
      const u32x4 kv = load16(ks + (kt * 32 + l32) * TL::LDK + k * 16 + hf * 8);
      st = Elem<T>::mfma32(as_vec8<T>(kv), qf[k], st);
    }
    __builtin_amdgcn_sched_barrier(0);
    // mask (diagonal / partial sub-tiles only) and raw row max
    const float shift = s.corr ? a.shift : 0.f;
    const bool need_mask = (s.nkeys < (kt + 1) * 32) || (!s.corr && s.key0 + kt * 32 + 31 > abs_first);
    if (need_mask) {
      const int key_lim = s.corr ? BN : qpos_abs - s.key0;  // causal: e <= key_lim
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int e = kt * 32 + (j >> 2) * 8 + hf * 4 + (j & 3);
        st[j] = (e < s.nkeys && e <= key_lim) ? st[j] : neg_inf();
      }
    }
    float mx = neg_inf();
#pragma unroll
    for (int j = 0; j < 16; j += 2) mx = fmaxf(fmaxf(mx, st[j]), st[j + 1]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_cand = fmaf(mx, c_pos, shift);  // -inf stays -inf (c_pos > 0)
    const bool upd = __ballot(m_cand > m_ref + kRescaleSlack) != 0ull;
    float alpha = 1.f;
    if (upd) {
      const float m_new = fmaxf(m_ref, m_cand);
      alpha = (m_new == neg_inf()) ? 1.f : __builtin_amdgcn_exp2f(m_ref - m_new);
      m_ref = m_new;
      l_run *= alpha;
    }
    const float bias = shift - ((m_ref == neg_inf()) ? 0.f : m_ref);
    vec8 pb[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      u32x4 w;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(st[u * 8 + 2 * i], c_pos, bias));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(st[u * 8 + 2 * i + 1], c_pos, bias));
        w[i] = pack2<T>(p0, p1);
        l_run = add_pair<T>(w[i], l_run);  // row sum of the rounded P used below
      }
      pb[u] = as_vec8<T>(w);
    }
    if (upd) {
#pragma unroll
      for (int dt = 0; dt < TL::DT; ++dt) {
#pragma unroll
        for (int j = 0; j < 16; ++j) o[dt][j] *= alpha;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // O^T += V^T . P^T.  The A operand (8 keys x 32 dims) comes from two
    // transposing LDS reads of the row-major V tile: keys
    // 32kt + 16u + 4hf + {0..3} and the same + 8, matching the key order of
    // this lane's P values.  Reads go in batches of 8 (4 MFMA operands): the
    // second batch is in flight while the first batch's MFMAs run.
    constexpr int PV_OPS = 2 * TL::DT;  // MFMAs of this slice: (u, dt)
    constexpr int PER_BATCH = 4;
    constexpr int BATCHES = (PV_OPS + PER_BATCH - 1) / PER_BATCH;
    // lane part of the address; the (kt, u, dt, +8 keys) parts are immediates
    const uint32_t vbase = lds_addr(vs) + ((hf * 4 + tr_row) * TL::LDVR + tr_col) * 2;
    u32x2 rb[2][8];
    auto issue_batch = [&](auto bc, u32x2 (&r)[8]) {
      constexpr int b = decltype(bc)::value;
      StaticFor<0, PER_BATCH>::run([&](auto qc) {
        constexpr int q = decltype(qc)::value;
        constexpr int op = b * PER_BATCH + q;
        if constexpr (op < PV_OPS) {
          constexpr int u = op / TL::DT, dt = op % TL::DT;
          constexpr int off = ((u * 16) * TL::LDVR + dt * 32) * 2;
          r[2 * q] = tr_read<off>(vbase + kt * 32 * TL::LDVR * 2);
          r[2 * q + 1] = tr_read<off + 8 * TL::LDVR * 2>(vbase + kt * 32 * TL::LDVR * 2);
        } else {
          r[2 * q] = u32x2{0u, 0u};
          r[2 * q + 1] = u32x2{0u, 0u};
        }
      });
    };
    auto run_batch = [&](auto bc, u32x2 (&r)[8]) {
      constexpr int b = decltype(bc)::value;
      StaticFor<0, PER_BATCH>::run([&](auto qc) {
        constexpr int q = decltype(qc)::value;
        constexpr int op = b * PER_BATCH + q;
        if constexpr (op < PV_OPS) {
          constexpr int u = op / TL::DT, dt = op % TL::DT;
          const u32x4 av = {r[2 * q][0], r[2 * q][1], r[2 * q + 1][0], r[2 * q + 1][1]};
          o[dt] = Elem<T>::mfma32(as_vec8<T>(av), pb[u], o[dt]);
        }
      });
    };
    issue_batch(std::integral_constant<int, 0>{}, rb[0]);
    tr_wait(rb[0]);
    StaticFor<0, BATCHES>::run([&](auto bc) {
      constexpr int b = decltype(bc)::value;
      if constexpr (b + 1 < BATCHES) issue_batch(std::integral_constant<int, b + 1>{}, rb[(b + 1) & 1]);
      run_batch(bc, rb[b & 1]);
      if constexpr (b + 1 < BATCHES) tr_wait(rb[(b + 1) & 1]);
    });
  };
  auto compute_step = [&](const Step& s, const uint16_t* stage) {
#pragma unroll
    for (int kt = 0; kt < TL::NTK; ++kt) {
      if (kt * 32 < s.nkeys || kt == 0) compute_slice(s, stage, kt);
    }
  };

  // ---- pipelined walk over the sub-tiles: the fills of step it+1 run while
  // step it is multiplied from the other stage; the loop is unrolled by two
  // so each half uses a fixed stage ----
  Step cur = next_step(0);
  if (n_steps > 0) fill_step(cur, stage0);
  fills_done();
  for (int it = 0; it < n_steps; it += 2) {
    {
      const bool more = it + 1 < n_steps;
      Step nxt{};
      if (more) {
        nxt = next_step(it + 1);
        fill_step(nxt, stage1);
      }
      compute_step(cur, stage0);
      fills_done();
      cur = nxt;
      if (!more) break;
    }
    {
      const bool more = it + 2 < n_steps;
      Step nxt{};
      if (more) {
        nxt = next_step(it + 2);
        fill_step(nxt, stage0);
      }
      compute_step(cur, stage1);
      fills_done();
      cur = nxt;
    }
  }

  // ---- normalise and store ----
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (!exists || pos >= a.out_rows) return;
  const float inv = (row_valid && l_tot > 0.f) ? 1.f / l_tot : 0.f;
  uint16_t* orow = a.out + (static_cast<int64_t>(h) * a.G + g) * a.o_hs + pos * a.o_rs;
#pragma unroll
  for (int dt = 0; dt < TL::DT; ++dt) {
#pragma unroll
    for (int jg = 0; jg < 4; ++jg) {
      const int d0 = dt * 32 + jg * 8 + hf * 4;
      u32x2 w;
      w[0] = pack2<T>(o[dt][jg * 4 + 0] * inv, o[dt][jg * 4 + 1] * inv);
      w[1] = pack2<T>(o[dt][jg * 4 + 2] * inv, o[dt][jg * 4 + 3] * inv);
      *reinterpret_cast<u32x2*>(orow + d0) = w;
    }
  }
}

template <typename T, int D, bool CORR>
int launch_attn(const AttnArgs& a, hipStream_t stream) {
  auto kernel = sparse_attn_kernel<T, D, CORR>;
  const int64_t wgs = static_cast<int64_t>(a.Hkv) * a.Nt * a.nchunk;
  if (wgs > 0x7fffffffLL) return fail(FPV2_ERR_UNSUPPORTED, "sparse_attention: grid too large");
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(wgs)), dim3(kThreads), 0, stream, a);
  return check_launch("sparse_attention");
}

template <typename T>
int dispatch_attn(int64_t D, bool corr, const AttnArgs& a, hipStream_t s) {
  switch (D) {
    case 64: return corr ? launch_attn<T, 64, true>(a, s) : launch_attn<T, 64, false>(a, s);
    case 96: return corr ? launch_attn<T, 96, true>(a, s) : launch_attn<T, 96, false>(a, s);
    case 128: return corr ? launch_attn<T, 128, true>(a, s) : launch_attn<T, 128, false>(a, s);
    case 256: return corr ? launch_attn<T, 256, true>(a, s) : launch_attn<T, 256, false>(a, s);
    default:
      return fail(FPV2_ERR_UNSUPPORTED, "head dimension must be one of (64, 96, 128, 256)");
  }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace
}  // namespace fpv2

extern "C" int fpv2_sparse_attention(const void* q, const void* k, const void* v,
                                     const void* pooled_k, const void* pooled_v,
                                     const int32_t* selected_ids, const int32_t* selected_counts,
                                     const int32_t* pruned_ids, const int32_t* pruned_counts,
                                     void* out, int dtype, const fpv2_attn_params* p,
                                     void* stream) {
  using namespace fpv2;
  if (!p || !q || !k || !v || !pooled_k || !pooled_v || !selected_ids || !selected_counts ||
      !pruned_ids || !pruned_counts || !out)
    return fail(FPV2_ERR_ARGUMENT, "sparse_attention: null argument");
  if (dtype != FPV2_BF16 && dtype != FPV2_F16)
    return fail(FPV2_ERR_UNSUPPORTED, "q, k, and v must share float16 or bfloat16 dtype");
  if (p->kv_heads <= 0 || p->query_heads <= 0 || p->query_heads % p->kv_heads)
    return fail(FPV2_ERR_ARGUMENT, "query heads must be divisible by KV heads");
  if (p->block_k <= 0 || p->tile_q <= 0 || p->num_blocks <= 0)
    return fail(FPV2_ERR_ARGUMENT, "sparse_attention: block_k, tile_q and num_blocks must be positive");
  if (p->padded_query_length <= 0 || p->padded_query_length % p->tile_q)
    return fail(FPV2_ERR_ARGUMENT, "q and k/v sequence lengths must be tile/block aligned");
  if (p->query_length <= 0 || p->query_length > p->padded_query_length)
    return fail(FPV2_ERR_ARGUMENT, "query_length must fit within padded q");
  if (p->out_rows < p->query_length || p->out_rows > p->padded_query_length)
    return fail(FPV2_ERR_ARGUMENT, "sparse_attention: out_rows must lie in [query_length, padded]");
  if (p->key_length <= 0 || p->key_length > p->num_blocks * p->block_k)
    return fail(FPV2_ERR_ARGUMENT, "key_length must fit within padded k/v");
  if (p->offset < 0 || p->offset + p->query_length > p->key_length)
    return fail(FPV2_ERR_ARGUMENT, "offset does not align queries within the key sequence");
  const int64_t strides[8] = {p->q_head_stride, p->q_row_stride, p->k_head_stride,
                              p->k_row_stride, p->v_head_stride, p->v_row_stride,
                              p->o_head_stride, p->o_row_stride};
  for (int i = 0; i < 8; ++i)
    if (strides[i] % 8) return fail(FPV2_ERR_UNSUPPORTED, "sparse_attention: strides must be multiples of 8 elements");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(pooled_k) ||
      !aligned16(pooled_v) || reinterpret_cast<uintptr_t>(out) % 8)
    return fail(FPV2_ERR_UNSUPPORTED, "sparse_attention: tensors must be 16-byte aligned");
  const int64_t G = p->query_heads / p->kv_heads;
  const int64_t D = p->head_dim;
  const int64_t Nt = p->padded_query_length / p->tile_q;
  const int64_t q_bytes = ((G - 1) * p->q_head_stride + (p->query_length - 1) * p->q_row_stride + D) * 2;
  const int64_t k_bytes = ((p->key_length - 1) * p->k_row_stride + D) * 2;
  const int64_t v_bytes = ((p->key_length - 1) * p->v_row_stride + D) * 2;
  const int64_t pooled_bytes = p->num_blocks * D * 2;
  if (q_bytes > kMaxRsrcBytes || k_bytes > kMaxRsrcBytes || v_bytes > kMaxRsrcBytes ||
      pooled_bytes > kMaxRsrcBytes)
    return fail(FPV2_ERR_UNSUPPORTED, "sparse_attention: a head group spans more than 2 GiB");
  if (p->q_row_stride < D || p->k_row_stride < D || p->v_row_stride < D || p->o_row_stride < D)
    return fail(FPV2_ERR_ARGUMENT, "sparse_attention: row strides must be >= head_dim");
  if (p->kv_heads * Nt * ((G * p->tile_q + kRows - 1) / kRows) > 0x7fffffffLL ||
      p->num_blocks * p->block_k > 0x7fffffffLL || G * p->tile_q > 0x7fffffffLL ||
      p->padded_query_length > 0x7fffffffLL)
    return fail(FPV2_ERR_UNSUPPORTED, "sparse_attention: sizes exceed 32-bit indexing");
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.pk = static_cast<const uint16_t*>(pooled_k);
  a.pv = static_cast<const uint16_t*>(pooled_v);
  a.ids = selected_ids;
  a.counts = selected_counts;
  a.pids = pruned_ids;
  a.pcounts = pruned_counts;
  a.out = static_cast<uint16_t*>(out);
  a.Hkv = static_cast<int>(p->kv_heads);
  a.G = static_cast<int>(G);
  a.Nt = static_cast<int>(Nt);
  a.Nb = static_cast<int>(p->num_blocks);
  a.Lq = static_cast<int>(p->query_length);
  a.out_rows = static_cast<int>(p->out_rows);
  a.Lk = static_cast<int>(p->key_length);
  a.offset = static_cast<int>(p->offset);
  a.bk = static_cast<int>(p->block_k);
  a.tq = static_cast<int>(p->tile_q);
  a.nchunk = static_cast<int>((G * p->tile_q + kRows - 1) / kRows);
  a.c_scale = static_cast<float>(p->scale * 1.4426950408889634);
  a.shift = static_cast<float>(__builtin_log2(static_cast<double>(p->block_k)));
  a.q_hs = p->q_head_stride;
  a.k_hs = p->k_head_stride;
  a.v_hs = p->v_head_stride;
  a.o_hs = p->o_head_stride;
  a.o_rs = p->o_row_stride;
  a.q_rs = static_cast<int>(p->q_row_stride);
  a.k_rs = static_cast<int>(p->k_row_stride);
  a.v_rs = static_cast<int>(p->v_row_stride);
  a.q_bytes = static_cast<uint32_t>(q_bytes);
  a.k_bytes = static_cast<uint32_t>(k_bytes);
  a.v_bytes = static_cast<uint32_t>(v_bytes);
  a.pooled_bytes = static_cast<uint32_t>(pooled_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool corr = p->mean_correction != 0;
  return dtype == FPV2_BF16 ? dispatch_attn<bf16_t>(p->head_dim, corr, a, s)
                            : dispatch_attn<f16_t>(p->head_dim, corr, a, s);
}
