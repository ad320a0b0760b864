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
//   * one workgroup = one (KV head, query tile, row chunk); the tile's G*tile_q
//     packed rows (row = g*tile_q + p) share the block lists, so the G query
//     heads of a KV head share every K/V load.  A workgroup has 4 waves
//     (128 rows, two workgroups per CU); D = 256 uses 8 waves for the same
//     rows, two per 32-row group, each owning half of the head dimension
//     for the products and half of each slice's keys for the softmax;
//   * each wave owns 32 query rows, two 16-row tiles; Q lives in VGPRs for
//     the whole walk;
//   * S^T = K . Q^T with v_mfma_f32_16x16x32_{bf16,f16} (2 x 2 tiles of 16
//     keys x 16 rows per 32-key slice): lane l owns query row l%16 of each
//     row tile and keys 4(l/16).. of each key tile, so row max/sum need two
//     lane exchanges and P feeds the PV MFMA without a transpose;
//   * O^T = V^T . P^T, each V^T fragment read once for both row tiles: the
//     rescale by exp2(m_old - m_new) is lane-local;
//   * K/V sub-tiles of 32 keys stream through a ring of NST LDS stages
//     filled by buffer_load_dwordx4 ... lds, NST-2 sub-tiles ahead of the
//     multiply; LDS rows are unpadded with an XOR swizzle of their
//     16-byte chunks, so K (ds_read_b128) and V (ds_read_b64_tr_b16, which
//     transposes on the way out) are read without bank conflicts and every
//     wave issues the same number of fills per stage;
//   * grid order puts the KV head in the low bits of the workgroup id, so the
//     round-robin dispatch over the 8 XCDs keeps one head per XCD L2 (for
//     Hkv = 8), and tiles run latest (longest) first.
#include <mutex>
#include <type_traits>

#include "fpv2_common.h"

namespace fpv2 {
namespace {

// ---- LDS access by inline asm (see fpv2_common.h) ----
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
// gfx950 transposing read (ds_read_b64_tr_b16): within each 16-lane group
// lane i receives element i%4 of the 8-byte chunks addressed by lanes
// i/4, i/4+4, i/4+8, i/4+12.
template <bool ASM, int OFF>
__device__ __forceinline__ u32x2 lds_read_tr(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field is 16 bits");
  if constexpr (ASM) {
    u32x2 r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
    return r;
  } else {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        reinterpret_cast<lds_s16x4*>(static_cast<uintptr_t>(addr + OFF)));
    return __builtin_bit_cast(u32x2, v);
  }
}
using ::fpv2::lgkm_wait;  // the single-register form, from fpv2_common.h
template <bool ASM, int N>
__device__ __forceinline__ void lgkm_wait(u32x2 (&r)[8]) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt is 4 bits");
  if constexpr (ASM)
    asm volatile("s_waitcnt lgkmcnt(%8)"
                 : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]),
                   "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7])
                 : "i"(N));
}
// In-place multiply; keeps a conditionally rescaled MFMA accumulator in its
// registers instead of a copy per branch.
__device__ __forceinline__ void scale_in_place(f32x4& acc, float f) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float x = acc[j];
    asm volatile("v_mul_f32 %0, %0, %1" : "+v"(x) : "v"(f));
    acc[j] = x;
  }
}

// max / sum of x over the four lanes l ^ {0, 16, 32, 48} that hold one row
// of a 16x16 accumulator: v_permlane16_swap_b32 then v_permlane32_swap_b32,
// whose two results hold x of both lanes of each pair in either order.
__device__ __forceinline__ float quad_max(float x) {
  // plain v_max_f32: the operands are MFMA results or -inf, never signalling
  // NaNs, so the canonicalising form fmaxf() would add is not needed
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  float m;
  asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(__uint_as_float(a[0])), "v"(__uint_as_float(a[1])));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(__uint_as_float(b[0])), "v"(__uint_as_float(b[1])));
  return m;
}
// (the pair sums are added in the same order in all four lanes, so they
// hold the same value)
__device__ __forceinline__ float quad_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
typedef float f32x2 __attribute__((ext_vector_type(2)));


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
  float inv_bk;   // 1 / block_k: the exact-phase weights' factor where the
                  // correction phase starts in the reference-free pass
  int64_t q_hs, k_hs, v_hs, o_hs, o_rs;
  int64_t pooled_hs;  // elements between KV heads of pk / pv
  int q_rs, k_rs, v_rs;
  uint32_t q_bytes, k_bytes, v_bytes, pooled_bytes;  // descriptor ranges
  // (last, so that the whole-tile kernel reads its other fields at the
  // offsets it had before the split existed)
  // Dense-tail split: the last split_tiles tiles run as nseg workgroups
  // each, over seg_steps consecutive sub-tiles of the tile's walk apiece,
  // writing unnormalised partials (O, l) and their scale m (the partial is
  // (O, l) * 2^m in the common scale of exp2(logit)) for merge_split_kernel.
  int split_tiles, nseg, seg_steps;
  float* ws_o;    // [item][seg][RW rows][D]
  float* ws_ml;   // [item][seg][RW rows][2]: m, l
};

// Workgroup barrier for data written to LDS by ds_write: it waits for this
// wave's LDS operations only.  __syncthreads() also waits for every
// outstanding global load, here the fills of the ring stages ahead.
__device__ __forceinline__ void barrier_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
template <typename V>
__device__ __forceinline__ V pick(bool c, V x, V y) {
  return c ? x : y;
}
__device__ __forceinline__ int clampi(int x, int lo, int hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

// LDS geometry of one K or V sub-tile: BN rows of ROWB bytes (D elements
// padded to a power of two), 16-byte chunk c of row r stored at chunk
// c ^ mask(r).  The masks make the 16 rows of a ds_read_b128 quarter-wave
// (16 keys, one chunk) hit 16 different 16-byte bank groups, and the 8 rows
// of each half of a transposing read (8 keys x 32 bytes of one d-tile) hit 8
// different 32-byte bank groups.
template <int D>
struct Geom {
  static constexpr int ROWB = D <= 64 ? 128 : (D <= 128 ? 256 : 512);
  static constexpr int RC = ROWB / 16;     // chunks per LDS row
  static constexpr int DG = D / 8;         // chunks holding data
  static constexpr int BN = 32;            // keys per sub-tile (one slice)
  static constexpr int TILE = BN * ROWB;   // bytes per K (or V) sub-tile
  static constexpr int STAGE = 2 * TILE;   // K then V
  static constexpr int JT = TILE / 1024;   // fill instructions (64 lanes x 16 B) per sub-tile
  static constexpr int RPI = 64 / RC;      // rows per fill instruction
  static constexpr int KS = D / 32;        // QK^T k-steps (32 dims each)
  static constexpr int DT = D / 16;        // O^T d-tiles (16 dims each)
  static __device__ __forceinline__ int kmask(int row) {
    return ROWB >= 256 ? (row & 15) : ((row >> 1) & 7);
  }
  // (even: chunk pairs stay pairs; rows of one 256-byte span apart)
  static __device__ __forceinline__ int vmask(int row) {
    return ROWB >= 256 ? ((row & 7) << 1) : (((row >> 1) & 3) << 1);
  }
};

// One K/V sub-tile of the walk: `nkeys` valid rows starting at key `key0`
// (exact phase) or at pruned-list entry `li` (correction phase).
struct Step {
  int corr;   // 0: exact keys of a selected block, 1: pooled entries of pruned blocks
  int li;     // first pruned-list entry (correction)
  int key0;   // first key (exact)
  int nkeys;  // valid rows in the sub-tile
};

// DS = 2: two waves share each 32-row group, each owning half of the head
// dimension: each multiplies its half of Q and K into a partial S.  Each
// wave of the pair also owns half of the slice's 32 keys: it sums the two
// partials of its 16 keys, computes their P and row sum, and hands its P to
// the partner through LDS at the same barrier as the partial S, so the
// softmax work is not repeated.  Each accumulates its half of O from both
// halves of P.  This keeps D = 256 at two waves per SIMD within 256
// registers.
// SEG: the launch of the split tiles' segments (every workgroup is one
// segment of one split tile), instantiated apart so that the whole-tile
// kernel's code carries nothing of it.
template <typename T, int D, bool CORR, int WAVES, int NST, int DS = 1, bool SEG = false>
__global__ __launch_bounds__(WAVES * 64, ((D <= 128 || DS == 2) ? 2 : 1)) void sparse_attn_kernel(AttnArgs a) {
  using GM = Geom<D>;
  constexpr int RT = 2;  // 16-row query tiles per wave (32 rows)
  constexpr int KT = 2;  // 16-key tiles per slice (32 keys)
  static_assert(DS == 1 || (DS == 2 && WAVES % 2 == 0 && GM::DT % 2 == 0 && GM::KS % 2 == 0),
                "D split in halves");
  // asm LDS reads unless a wave's registers do not hold them (D = 256 without
  // the split), where the compiler schedules its LDS reads (see lds_read_b128).
  constexpr bool kAsm = D <= 128 || DS == 2;
  constexpr int DT = GM::DT / DS;  // 16-wide output d-tiles of this wave
  constexpr int KSQ = GM::KS / DS; // 32-deep QK k-steps of this wave
  constexpr int KR = 2 * KSQ;      // K fragment reads per slice: (k-step, key tile)
  // DS = 2: the first wave of a pair owns key tile 0 (keys 0-15 of each
  // slice), the second key tile 1 (keys 16-31).
  constexpr bool KSPLIT = DS == 2;
  using vec8 = typename Elem<T>::vec8;
  constexpr int BN = GM::BN;
  constexpr int ROWB = GM::ROWB;
  constexpr int RW = WAVES / DS * 32;     // packed query rows per workgroup
  constexpr int NIK = GM::JT / WAVES;     // fill instructions per wave per sub-tile
  constexpr int NI = 2 * NIK;             // ... per stage (K then V)
  static_assert(GM::JT % WAVES == 0, "fills must split evenly over the waves");
  static_assert(NST >= 2 && NI * (NST - 2) <= 63, "vmcnt range");
  // the stage ring, then (DS = 2) 4 KiB per wave for its partner: bytes
  // [0, 1024) its P (16 bytes per lane), [1024, 1536) two floats per lane
  // (row max or row sum of both row tiles), [2048, 4096) its partial S of
  // the partner's key tile
  __shared__ __align__(1024) uint8_t smem[NST * GM::STAGE + (DS == 2 ? WAVES * 4096 : 0)];
  uint8_t* const xbuf = smem + NST * GM::STAGE;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int l16 = lane & 15;
  const int grp = lane >> 4;  // 16-lane group: keys 4*grp.. of each key tile

  // ---- workgroup -> (KV head, tile, row chunk); latest tiles first ----
  // Whole tiles: [0, Nt - split_tiles).  Segments (SEG): seg of the split
  // tiles [Nt - split_tiles, Nt).  The KV head is in the low bits.
  const int bid = blockIdx.x;
  const int h = bid % a.Hkv;
  int rest = bid / a.Hkv;
  const int seg = SEG ? rest % a.nseg : -1;
  if constexpr (SEG) rest /= a.nseg;
  const int chunk = rest % a.nchunk;
  const int t = (SEG ? a.Nt : a.Nt - a.split_tiles) - 1 - rest / a.nchunk;
  const int abs_first = a.offset + t * a.tq;
  const int last_local = min((t + 1) * a.tq, a.Lq);
  const int abs_last = a.offset + last_local - 1;

  // ---- this lane's query rows: row l16 of each of the wave's two 16-row
  // tiles (the S^T / O^T column the lane holds) ----
  const int R = a.G * a.tq;
  const int rwave = wave % (WAVES / DS);  // 32-row group of this wave
  const int dhalf = wave / (WAVES / DS);  // part of the head dimension (DS = 2)
  bool exists[RT], row_valid[RT];
  int g[RT], pos[RT], qpos_abs[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int prow = chunk * RW + rwave * 32 + rt * 16 + l16;
    exists[rt] = prow < R;
    g[rt] = 0;
    pos[rt] = 0;
    if (exists[rt]) {
      g[rt] = prow / a.tq;
      pos[rt] = t * a.tq + (prow - g[rt] * a.tq);
    }
    row_valid[rt] = exists[rt] && pos[rt] < a.Lq;
    qpos_abs[rt] = a.offset + pos[rt];
  }

  // bfloat16 (8 exponent bits, like float32) takes the reference-free first
  // pass: Q is loaded pre-multiplied by c = scale*log2(e) (one rounding to
  // bf16 per element, at most 2^-9 relative), so S = K.Q'^T is already in
  // log2 units and P = exp2(S) needs no VALU before the exp; rows whose sums
  // or outputs leave the float32 range walk again with an online reference.
  // float16 P (5 exponent bits) needs a reference: its first pass takes
  // each row's max over its first slice and P = exp2(s*c - m_ref).
  constexpr bool kFree = std::is_same<T, bf16_t>::value;
  // Q^T fragments (the B operand): lane l holds 8 consecutive dims
  // 32k + 8*grp.. of its row in each row tile
  vec8 qf[RT][KSQ];
  {
    const rsrc_t qr = make_rsrc(a.q + static_cast<int64_t>(h) * a.G * a.q_hs, a.q_bytes);
    // float16: the softmax folds the scale into one FMA per logit and needs
    // a positive factor: for scale < 0 the queries are negated instead
    // (s*c = (-s)*(-c)).
    const uint32_t sign = (!kFree && a.c_scale < 0.f) ? 0x80008000u : 0u;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const uint32_t qoff =
          row_valid[rt]
              ? static_cast<uint32_t>((g[rt] * a.q_hs + static_cast<int64_t>(pos[rt]) * a.q_rs + grp * 8) * 2)
              : kOOB;
#pragma unroll
      for (int k = 0; k < KSQ; ++k) {
        u32x4 v = buf_load16(qr, qoff + (row_valid[rt] ? (dhalf * KSQ + k) * 64 : 0));
        if constexpr (kFree) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            v[e] = pack2<T>(__uint_as_float(v[e] << 16) * a.c_scale,
                            __uint_as_float(v[e] & 0xffff0000u) * a.c_scale);
        } else {
          v ^= sign;
        }
        qf[rt][k] = as_vec8<T>(v);
      }
    }
  }
  // factor from S to log2 units (1 when Q carries it)
  const float c_pos = kFree ? 1.f : fmaxf(fabsf(a.c_scale), 1e-30f);

  // ---- block lists of (h, t), clipped as kernel.py:555-558 ----
  // The counts and the first 64 entries of both lists are requested together
  // (one memory round trip, alongside Q); the walk's set-up below reads them
  // from registers, so a workgroup with short lists starts filling after two
  // round trips instead of one per dependent step.
  const int Nb = a.Nb;
  const int64_t list_row = static_cast<int64_t>(h) * a.Nt + t;
  const int32_t* ids = a.ids + list_row * Nb;
  const int32_t* pids = a.pids + list_row * Nb;
  const int cnt_raw = a.counts[list_row];
  const int pcnt_raw = CORR ? a.pcounts[list_row] : 0;
  const int id_lane = clampi(ids[min(lane, Nb - 1)], 0, Nb - 1);  // entry `lane`
  const int sel_count = clampi(cnt_raw, 0, Nb);
  const int pr_count = CORR ? clampi(pcnt_raw, 0, Nb) : 0;
  const int subs = (a.bk + BN - 1) / BN;

  // The walk stops at the first listed block that starts after the tile's
  // last row (kernel.py:252): one ballot per 64 entries, the first 64 from
  // registers, later ones four loads at a time.
  int li_end = sel_count;
  {
    const uint64_t m0 = __ballot(lane < sel_count && id_lane * a.bk > abs_last);
    if (m0 != 0ull) {
      li_end = static_cast<int>(__builtin_ctzll(m0));
    } else {
      for (int base = 64; base < sel_count; base += 256) {
        bool found = false;
        int idv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int li = base + 64 * j + lane;
          idv[j] = li < sel_count ? clampi(ids[li], 0, Nb - 1) : 0;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int li = base + 64 * j + lane;
          const uint64_t m = __ballot(li < sel_count && idv[j] * a.bk > abs_last);
          if (!found && m != 0ull) {
            li_end = base + 64 * j + static_cast<int>(__builtin_ctzll(m));
            found = true;
          }
        }
        if (found) break;
      }
    }
  }
  // Exact-phase sub-tiles: every sub-tile of the blocks before li_end, the
  // last block trimmed at the tile's last row; sub-tiles of other blocks that
  // start past it (only in non-ascending lists) are skipped as empty.
  int n_sel = 0;
  if (li_end > 0) {
    const int last_blk = li_end <= 64 ? __builtin_amdgcn_readlane(id_lane, li_end - 1)
                                      : clampi(ids[li_end - 1], 0, Nb - 1);
    n_sel = (li_end - 1) * subs + min(subs, (abs_last - last_blk * a.bk) / BN + 1);
  }
  const int n_corr = CORR ? (pr_count + BN - 1) / BN : 0;
  const int n_steps = n_sel + n_corr;

  // Exact steps are described 64 at a time: lane j of a window holds the
  // first key and valid-row count of step win_base + j, computed in one
  // vector pass from the selected list, and a step reads its pair with two
  // readlanes.  With correction, the list entries of the next window are
  // loaded one window ahead (win_next, raw; entries past the list row read
  // as 0): a window computed from a load issued in the same step waits for
  // every fill in flight (vmcnt(0)).  Without correction the kernel has no
  // register for win_next (it would spill in the slice loop) and loads each
  // window when it is reached.  Correction steps follow from the step index.
  int win_base = 0, win_key0 = 0, win_nk = 0;
  auto window_entry = [&](int it, int blk) {
    const int li = it / subs;
    const int sub = it - li * subs;
    const int key0 = blk * a.bk + sub * BN;
    const int n = min(min(a.bk - sub * BN, BN), a.Lk - key0);
    win_key0 = key0;
    win_nk = (it >= n_sel || key0 > abs_last || n < 0) ? 0 : n;
  };
  const rsrc_t idr = make_rsrc(ids, static_cast<uint32_t>(Nb) * 4u);
  auto load_window = [&](int base) {  // raw entry of step base + lane
    return static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(idr, ((base + lane) / subs) * 4, 0, 0));
  };
  // A workgroup walks steps [s_lo, s_hi): all of the tile's, or a
  // segment's seg_steps of them.
  const int s_lo = SEG ? min(seg * a.seg_steps, n_steps) : 0;
  const int s_hi = SEG ? min(s_lo + a.seg_steps, n_steps) : n_steps;
  // The window holding step s: the first window's entries come from id_lane
  // (its steps cover at most the first 64 entries), later ones are loaded.
  int win_next = 0;
  auto start_windows = [&](int s) {
    win_base = SEG ? (s / 64) * 64 : 0;
    if (!SEG || win_base == 0) {
      window_entry(lane, __builtin_amdgcn_ds_bpermute((lane / subs) * 4, id_lane));
    } else {
      const int li = (win_base + lane) / subs;  // < li_end when the step is < n_sel
      window_entry(win_base + lane, win_base + lane < n_sel ? clampi(ids[min(li, Nb - 1)], 0, Nb - 1) : 0);
    }
    if constexpr (CORR) win_next = load_window(win_base + 64);
  };
  start_windows(s_lo);
  // A walk covers steps [walk_it, walk_end): the workgroup's, or (the
  // reference-free pass with correction) its exact steps, then its
  // correction steps.
  int walk_it = s_lo, walk_end = s_hi;
  // KIND: 0 a walk of both kinds of steps, 1 of exact steps only, 2 of
  // correction steps only.  (A walk of correction steps has no window to
  // carry: where one walk served both, the compiler waited for the window
  // load with vmcnt(0) before copying its register at every correction
  // step, which drained the fills in flight.)
  auto next_step = [&](auto kind_c) -> Step {
    constexpr int KIND = decltype(kind_c)::value;
    Step s{0, 0, 0, 0};  // past the end: an empty sub-tile (all-zero fill)
    const int it = walk_it++;
    if (KIND != 2 && it < n_sel && it < walk_end) {
      if (it - win_base >= 64) {
        win_base += 64;
        if constexpr (CORR) {
          window_entry(win_base + lane, win_base + lane < n_sel ? clampi(win_next, 0, Nb - 1) : 0);
          win_next = load_window(win_base + 64);
        } else {
          const int li = (win_base + lane) / subs;  // < li_end when the step is < n_sel
          window_entry(win_base + lane, win_base + lane < n_sel ? clampi(ids[li], 0, Nb - 1) : 0);
        }
      }
      s.key0 = __builtin_amdgcn_readlane(win_key0, it - win_base);
      s.nkeys = __builtin_amdgcn_readlane(win_nk, it - win_base);
    } else if (KIND != 1 && it < walk_end) {
      s.corr = 1;
      s.li = (it - n_sel) * BN;
      s.nkeys = min(pr_count - s.li, BN);
    }
    return s;
  };

  // ---- global -> LDS fills (buffer_load_dwordx4 ... lds) ----
  // Fill instruction i of this wave covers rows [jj*RPI, (jj+1)*RPI) of the K
  // (i < NIK) or V sub-tile, jj = wave + (i % NIK) * WAVES; lane -> chunk
  // lane % RC of row jj*RPI + lane / RC, holding data chunk c = that ^ mask.
  const uint16_t* const kh = a.k + h * a.k_hs;
  const uint16_t* const vh = a.v + h * a.v_hs;
  const uint16_t* const pkh = a.pk + h * a.pooled_hs;
  const uint16_t* const pvh = a.pv + h * a.pooled_hs;
  auto fill_row = [&](int i, int ln) { return (wave + (i % NIK) * WAVES) * GM::RPI + ln / GM::RC; };
  auto fill_chunk = [&](int i, int row, int ln) {
    return (ln % GM::RC) ^ (i < NIK ? GM::kmask(row) : GM::vmask(row));
  };
  // The rare partial and correction fills recompute rows and chunks from an
  // opaque copy of the lane id, so that their per-lane constants are not
  // hoisted out of the walk to occupy registers for its whole length.
  auto opaque_lane = [&]() {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    return ln;
  };
  // Byte offset of the lane's chunk relative to the sub-tile's first key
  // (kOOB: a pad chunk past D).  Constant over the walk: an exact fill adds
  // its sub-tile's offset as the instruction's scalar offset.
  uint32_t pre[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int row = fill_row(i, lane);
    const int c = fill_chunk(i, row, lane);
    const int rs = i < NIK ? a.k_rs : a.v_rs;
    pre[i] = c < GM::DG ? static_cast<uint32_t>((row * rs + c * 8) * 2) : kOOB;
  }
  const uint32_t smem_lds = lds_addr(smem);
  // Correction fills take their pooled rows' block ids from cid: the
  // pruned-list entries li + fill_row(j, lane) of the next correction step
  // (the first one's, loaded at set-up, through the exact phase).  A
  // correction fill computes its addresses from cid, then loads the next
  // step's entries into cid, then issues its fills.  The fills of every kind
  // of step are issued on one path after that point: the compiler's wait
  // analysis does not tell branches apart, and a load that some path does
  // not follow with the step's fills (or that is consumed at once) gets a
  // vmcnt(0) wait before its use, draining every fill in flight.  Followed
  // by the fills, the loads are known to be complete after the fills_done()
  // wait before their use.  Raw buffer loads over the rest of the list row:
  // entries past the row read as 0; values are clamped where they are used.
  int cid[NIK];
  auto load_cids = [&](int li) {
    const rsrc_t pr = make_rsrc(pids + li, static_cast<uint32_t>(max(Nb - li, 0)) * 4u);
#pragma unroll
    for (int j = 0; j < NIK; ++j)
      cid[j] = CORR ? static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(pr, fill_row(j, lane) * 4, 0, 0)) : 0;
  };
  // (the first correction step of the workgroup's range)
  load_cids(max(s_lo - n_sel, 0) * BN);
  auto fill_step = [&](const Step& s, int stage, auto kind_c) {
    constexpr int KIND = decltype(kind_c)::value;
    typedef __attribute__((address_space(3))) void* lds_ptr;
    // (a lambda returning an LDS pointer would drop the kernel from the host
    // pass, so the destination is spelled out at each fill)
    uint8_t* const sp = smem + stage * GM::STAGE;
    // NI fills with per-lane offsets vo and the uniform offsets sk (K) and
    // sv (V).  (The builtin's arguments are plain locals: some argument
    // expressions drop the kernel's host-side stub without a diagnostic.)
    auto issue = [&](const uint32_t (&vo)[NI], uint32_t sk, uint32_t sv, rsrc_t rk, rsrc_t rv) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const rsrc_t r = i < NIK ? rk : rv;
        const uint32_t o = vo[i];
        const uint32_t so = i < NIK ? sk : sv;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            r, (lds_ptr)(sp + (i < NIK ? 0 : GM::TILE) + (wave + (i % NIK) * WAVES) * 1024), 16, o, so,
            0, 0);
      }
    };
    // (uniform: it selects the kind of fill)
    const bool corr = CORR && __builtin_amdgcn_readfirstlane(s.corr) != 0;
    // An exact fill takes its sub-tile's first key as the scalar offsets (a
    // lane past the sub-tile's keys or past D has the offset kOOB, which
    // stays out of range with them).
    const uint32_t kb = static_cast<uint32_t>(s.key0 * a.k_rs * 2);
    const uint32_t vb = static_cast<uint32_t>(s.key0 * a.v_rs * 2);
    auto corr_offsets = [&](uint32_t (&off)[NI]) {  // pooled rows of the pruned blocks
      const int ln = opaque_lane();
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int row = fill_row(i, ln);
        const int c = fill_chunk(i, row, ln);
        const int blk = clampi(cid[i % NIK], 0, Nb - 1);  // entry s.li + row
        const bool ok = row < s.nkeys && c < GM::DG;
        off[i] = ok ? static_cast<uint32_t>((blk * D + c * 8) * 2) : kOOB;
      }
    };
    if constexpr (KIND != 0 || !CORR) {
      // A walk of one kind of step: each kind of fill issues its own, so
      // that the full exact fill, the common one, takes the constant
      // offsets as they are.  (The empty asm statements that end the two
      // exact paths differ, so the compiler does not merge their fills
      // behind copies of the offsets.)
      if (!corr) {
        const rsrc_t rk = make_rsrc(kh, a.k_bytes);
        const rsrc_t rv = make_rsrc(vh, a.v_bytes);
        if (s.nkeys == BN) {  // full sub-tile
          issue(pre, kb, vb, rk, rv);
          asm volatile("; full sub-tile");
        } else {  // partial (end of the keys or of a block) or empty
          const int ln = opaque_lane();
          uint32_t vo[NI];
#pragma unroll
          for (int i = 0; i < NI; ++i) vo[i] = fill_row(i, ln) < s.nkeys ? pre[i] : kOOB;
          issue(vo, kb, vb, rk, rv);
          asm volatile("; partial sub-tile");
        }
      } else {
        uint32_t off[NI];
        corr_offsets(off);
        load_cids(s.li + BN);  // the next correction step's entries
        issue(off, 0u, 0u, make_rsrc(pkh, a.pooled_bytes), make_rsrc(pvh, a.pooled_bytes));
      }
    } else {
      // Both kinds in one walk: every fill is issued on one path after the
      // next correction entries are loaded (see above).  Issued per kind,
      // the entries' registers are copied at each exact step with a wait
      // that covers the previous step's fills.
      uint32_t vo[NI];
      if (!corr) {
        if (s.nkeys == BN) {
#pragma unroll
          for (int i = 0; i < NI; ++i) vo[i] = pre[i];
        } else {
          const int ln = opaque_lane();
#pragma unroll
          for (int i = 0; i < NI; ++i) vo[i] = fill_row(i, ln) < s.nkeys ? pre[i] : kOOB;
        }
      } else {
        corr_offsets(vo);
      }
      if (corr) load_cids(s.li + BN);
      // (descriptors built from selected values: a select between two
      // descriptors, or between two captured variables, is lowered through
      // memory)
      issue(vo, corr ? 0u : kb, corr ? 0u : vb, make_rsrc(pick(corr, pkh, kh), pick(corr, a.pooled_bytes, a.k_bytes)),
            make_rsrc(pick(corr, pvh, vh), pick(corr, a.pooled_bytes, a.v_bytes)));
    }
  };
  // Fills run LA = NST-2 sub-tiles ahead of the multiply, so that the stage
  // of the previous sub-tile, whose last slice is still being multiplied by
  // V (see the slice pipeline below), is not refilled yet.  The fills of a
  // stage are complete once at most the LA-1 younger stages' fills (NI
  // instructions each) are outstanding in this wave, and in every wave after
  // the barrier.
  constexpr int LA = NST - 2;
  static_assert(LA >= 1, "the slice pipeline needs NST >= 3");
  auto fills_done = [&]() {
    vm_wait<NI * (LA - 1)>();
    __builtin_amdgcn_s_barrier();
  };

  // ---- accumulators ----
  // Online softmax in log2 units with a lazily updated reference max m_ref:
  // P = exp2(s*c + shift - m_ref) may exceed 1 by up to 2^kRescaleSlack, and
  // O / l are rescaled only when some row's max grows past that, so the
  // common case costs no rescale at all.  The result O / l is unchanged.
  constexpr float kRescaleSlack = 8.0f;
  // O^T tiles: o[dt][rt] holds dims 16dt + 4grp + 0..3 of the lane's row of
  // row tile rt (a 16x16 accumulator of v_mfma_f32_16x16x32)
  f32x4 o[DT][RT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) o[dt][rt] = f32x4{};
  }
  float m_ref[RT];
  // Derived from m_ref, updated only when it changes: the exp2 bias
  // (-m_ref, 0 while no key has been seen) and the rescale threshold.  The
  // kernels without correction, and those with D = 256, are at the register
  // limit and recompute them per slice instead of keeping two more live values.
  constexpr bool kKeepRef = CORR && D <= 128;
  float neg_m[RT], m_thr[RT], l_run[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m_ref[rt] = neg_inf();
    neg_m[rt] = 0.f;
    m_thr[rt] = neg_inf();
    l_run[rt] = 0.f;
  }
  auto bias_of_ref = [&](int rt) {
    return kKeepRef ? neg_m[rt] : ((m_ref[rt] == neg_inf()) ? 0.f : -m_ref[rt]);
  };
  auto thr_of_ref = [&](int rt) { return kKeepRef ? m_thr[rt] : m_ref[rt] + kRescaleSlack; };

  // LDS read addresses relative to a slice (32 keys of a stage).
  // K, the A operand of S^T = K . Q'^T: lane l reads key row l16 (+16 rows,
  // an immediate offset, for key tile 1) and the 16-byte chunk 4k + grp of
  // k-step k, stored at chunk (4k + grp) ^ kmask = 4k ^ (grp ^ kmask):
  // kbase ^ 64k.  V^T, the A operand of O^T = V^T . P^T: lane i of 16-lane
  // group grp receives the 4 keys 4grp.. (and 16 + 4grp..) of dim 16dt + i;
  // lane m of the group addresses key row 4grp + m/4 and the 8 bytes of dims
  // 16dt + 4(m%4).., chunk (2dt + (m%4)/2) ^ vmask = 2dt ^ ((m%4)/2 ^ vmask):
  // vbase ^ 32dt.  The XOR terms touch address bits 4-7 only, and slice
  // offsets (whole stages) and the key-tile and D-half offsets lie above
  // them.  (DS = 2: this wave's k-steps and d-tiles start KSQ*64 and DT*32
  // bytes along the row, and its own key tile, read first, 16*dhalf rows
  // in; the partner's tile is 16 rows away, an XOR of the 16*ROWB bit.)
  const int km = GM::kmask(l16);
  const int own = KSPLIT ? 16 * dhalf : 0;
  const uint32_t kbase = smem_lds + (own + l16) * ROWB + (grp ^ km) * 16 + dhalf * KSQ * 64;
  const int vrow = 4 * grp + (l16 >> 2);
  const int vm = GM::vmask(vrow);
  const uint32_t vbase = smem_lds + GM::TILE + (own + vrow) * ROWB + (((l16 & 3) >> 1) ^ vm) * 16 +
                         (l16 & 1) * 8 + dhalf * DT * 32;
  // Walks whose ring stage is known at compile time (the 4-wave shape on
  // whole tiles) read K and V at per-lane addresses computed once, with the
  // stage in the instruction's immediate offset: the XOR terms touch
  // address bits 4-7 only, which a stage offset (a multiple of the stage
  // size) leaves alone.
  constexpr bool kImm = !KSPLIT && !SEG;
  static_assert(!kImm || (NST - 1) * GM::STAGE + 16 * ROWB < 65536, "ds offset field is 16 bits");
  uint32_t kx[KSQ], vx[DT];
  if constexpr (kImm) {
#pragma unroll
    for (int ks = 0; ks < KSQ; ++ks) kx[ks] = kbase ^ (64 * ks);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) vx[dt] = vbase ^ (32 * dt);
  }
  using NoStage = std::integral_constant<int, -1>;

  // ---- slice pipeline ----
  // A slice is 32 keys of a sub-tile.  Each slice passes two pipeline
  // stages, one process() call apart, so that every stage pairs MFMA work
  // with VALU work of another slice:
  //   A: S^T = K . Q'^T of slice n      ||  exp2 / pack / row sum of 6 of
  //                                         the 8 key pairs of slice n-1
  //   B: O^T += V^T . P^T of slice n-1  ||  the last 2 key pairs (during the
  //                                         MFMAs of the first row tile),
  //                                         mask and row max of slice n
  //   C: (rare) rescale of O and l when slice n raises the reference max.
  // A wave keeps its matrix pipe busy during its own softmax; the order of
  // issue within A and B is fixed in source order, each piece of VALU work
  // consumed by an empty asm statement so the compiler cannot regroup it.
  struct Slice {
    int corr;       // pooled correction rows (logit shift, no causal mask)
    int key0;       // first key (exact slices)
    int nkeys;      // valid rows from the slice start (may exceed 32)
    uint32_t off;   // byte offset of the slice within the stage ring
  };
  auto make_slice = [&](const Step& s, int stage, int kt) {
    Slice r;
    r.corr = s.corr;
    r.key0 = s.key0 + kt * 32;
    r.nkeys = s.nkeys - kt * 32;
    r.off = static_cast<uint32_t>(stage * GM::STAGE + kt * 32 * ROWB);
    return r;
  };
  // S^T of the slice between stages A and B of the pipeline (masked, its max
  // folded into m_ref), in one of two buffers that alternate between slices:
  // s[rt][kt] holds keys 16kt + 4grp + 0..3 of the lane's row of row tile
  // rt.  (DS = 2: s[rt][0] holds the wave's own key tile, s[rt][1] the
  // partner's, whose partial this wave hands over.)
  f32x4 s_buf[2][RT][KT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) s_buf[0][rt][kt] = s_buf[1][rt][kt] = f32x4{};
  }
  Slice p_pend{0, 0, 0, 0u};

  // issue-order tuning of the slice pipeline (see process_m)
#ifndef FPV2_EXP_A
#define FPV2_EXP_A 6
#endif
  // exp pairs of the pending slice in stage A (the first row tile's four,
  // then the second's); the rest are spread over the first row tile's PV
  // MFMAs of the first V batch
  constexpr int kExpA = FPV2_EXP_A;
  static_assert(kExpA >= 4 && kExpA <= 8, "the first row tile's P is built in stage A");
  constexpr int PER_BATCH = 4;  // V^T fragments (d-tiles) per batch of 8 transposing reads
  constexpr int BATCHES = (DT + PER_BATCH - 1) / PER_BATCH;
  // V^T fragment of d-tile dt: the keys 4grp.. (slots 0-3 of the PV
  // contraction) and 16 + 4grp.. (slots 4-7), as the P words are ordered.
  // (DS = 2: slots 0-3 are the wave's own key tile, 16*dhalf + 4grp.., and
  // slots 4-7 the partner's, so the second read flips the 16-row offset.)
  auto issue_v = [&](uint32_t va, auto bc, u32x2 (&r)[8], auto sp_c) {
    constexpr int b = decltype(bc)::value;
    constexpr int SP = decltype(sp_c)::value;  // the slice's stage, if known
    StaticFor<0, PER_BATCH>::run([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      constexpr int dt = b * PER_BATCH + q;
      if constexpr (dt < DT && kImm && SP >= 0) {
        r[2 * q] = lds_read_tr<kAsm, SP * GM::STAGE>(vx[dt]);
        r[2 * q + 1] = lds_read_tr<kAsm, SP * GM::STAGE + 16 * ROWB>(vx[dt]);
      } else if constexpr (dt < DT) {
        const uint32_t addr = va ^ (32 * dt);
        r[2 * q] = lds_read_tr<kAsm, 0>(addr);
        if constexpr (KSPLIT) r[2 * q + 1] = lds_read_tr<kAsm, 0>(addr ^ (16 * ROWB));
        else r[2 * q + 1] = lds_read_tr<kAsm, 16 * ROWB>(addr);
      } else {
        r[2 * q] = u32x2{0u, 0u};
        r[2 * q + 1] = u32x2{0u, 0u};
      }
    });
  };
  // process<HN, HP, B>(nw): stage A and B for the new slice nw (if HN, into
  // s_buf[B]) and the pending slice (if HP, in s_buf[1-B]); nw becomes
  // pending.
  auto needs_mask = [&](const Slice& nw) {
    return nw.nkeys < 32 || (!nw.corr && nw.key0 + 31 > abs_first);
  };
  // MODE: how the new slice's row max is used (see the walk below)
  //   0  not computed (the fixed reference of the first pass),
  //   1  sets the reference (the first slice of the first pass),
  //   2  online reference with rescale (the exact pass).
  // SN, SP: the ring stages of the new and the pending slice when known at
  // compile time (-1: from the slices' offsets).
  auto process_m = [&](auto hn_c, auto hp_c, auto b_c, auto mask_c, auto mode_c, auto sn_c, auto sp_c,
                       const Slice& nw) {
    constexpr int SN = decltype(sn_c)::value;
    constexpr bool HN = decltype(hn_c)::value;
    constexpr bool HP = decltype(hp_c)::value;
    constexpr int B = decltype(b_c)::value;
    constexpr bool MASK = decltype(mask_c)::value;
    constexpr int MODE = decltype(mode_c)::value;
    constexpr bool MAX = HN && MODE != 0;
    // the reference-free first pass: P = exp2(S) (the correction slices'
    // shift is applied once, as a rescale between the exact and the
    // correction walks)
    constexpr bool RAW = kFree && MODE == 0;
    f32x4(&s_new)[RT][KT] = s_buf[B];
    f32x4(&s_old)[RT][KT] = s_buf[1 - B];
    constexpr int KW = KR < 4 ? KR : 4;  // K fragment reads in flight
    const uint32_t va = vbase + p_pend.off;
    const uint32_t ka = kbase + nw.off;
    u32x2 vb[2][8];
    u32x4 kf[KR];
    vec8 pb[RT];
    // K fragment read i: k-step i / 2, key tile i % 2 (DS = 2: tile 0 is the
    // wave's own, 16*dhalf rows in)
    auto read_k = [&](auto ic) {
      constexpr int i = decltype(ic)::value;
      constexpr int ks = i / 2, kt = i % 2;
      if constexpr (KSPLIT) return lds_read_b128<kAsm, 0>(ka ^ (64 * ks + kt * 16 * ROWB));
      else if constexpr (kImm && SN >= 0) return lds_read_b128<kAsm, SN * GM::STAGE + kt * 16 * ROWB>(kx[ks]);
      else return lds_read_b128<kAsm, kt * 16 * ROWB>(ka ^ (64 * ks));
    };

    // ---- stage A ----
    // Wave priority: a wave in the VALU-heavy stage A yields issue to the
    // other wave of its SIMD when that one is in stage B (PV MFMAs, light
    // VALU) or in its fills, which keeps the matrix pipe fed.
    __builtin_amdgcn_s_setprio(0);
    // A window of KW K fragments of the new slice, then V^T batch 0 of the
    // pending slice; each group of QK MFMAs issues the read KW fragments
    // ahead.  Reads complete in order, so fragment i is ready once at most
    // the reads issued after it are outstanding.  The exp section of the
    // pending slice is spread over the QK MFMAs in source order; an empty asm
    // that consumes each piece keeps the compiler from regrouping them.
    if constexpr (HN) {
      StaticFor<0, KW>::run([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        kf[i] = read_k(ic);
      });
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) s_new[rt][kt] = f32x4{};
      }
    }
    // V^T batch 0 after the first K window: those K reads do not wait behind it
    if constexpr (HP) issue_v(va, std::integral_constant<int, 0>{}, vb[0], sp_c);
    constexpr int NV0 = HP ? 2 * PER_BATCH : 0;  // reads of batch 0
    float bias[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      bias[rt] = 0.f;
      // (the logit shift of correction slices selected as scalar bits, so
      // the add takes it from an SGPR)
      if constexpr (HP && !RAW)
        bias[rt] = bias_of_ref(rt) +
                   __uint_as_float(__builtin_amdgcn_readfirstlane(p_pend.corr ? __float_as_uint(a.shift) : 0u));
    }
    // P words of the pending slice: w[rt][e] packs keys 2e, 2e + 1 of the
    // PV contraction slots (slot 4kt + r: key 16kt + 4grp + r).  DS = 2: the
    // wave computes its own key tile's words (e = 0, 1); the partner's
    // arrive through LDS as e = 2, 3.
    u32x4 w[RT];
    constexpr int NP = KSPLIT ? 2 * RT : 4 * RT;  // exp pairs per slice
    auto exp_pair = [&](auto fc) {
      constexpr int f = decltype(fc)::value;
      constexpr int rt = f / (NP / RT), e = f % (NP / RT);
      constexpr int kt = e / 2, r0 = 2 * (e % 2);
      const float x0 = RAW ? s_old[rt][kt][r0] : fmaf(s_old[rt][kt][r0], c_pos, bias[rt]);
      const float x1 = RAW ? s_old[rt][kt][r0 + 1] : fmaf(s_old[rt][kt][r0 + 1], c_pos, bias[rt]);
      const float p0 = __builtin_amdgcn_exp2f(x0);
      const float p1 = __builtin_amdgcn_exp2f(x1);
      const uint32_t word = pack2<T>(p0, p1);
      l_run[rt] = add_pair<T>(word, l_run[rt]);  // row sum of the rounded P used below
      w[rt][e] = word;
      asm volatile("" ::"v"(word));
    };
    if constexpr (HN) {
      constexpr int EA = KSPLIT ? NP : kExpA;  // (DS = 2: all before the exchange)
      StaticFor<0, KR>::run([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        // reads issued after K fragment i: the rest of the first window, the
        // V batch, and the fragments issued by earlier MFMA groups
        constexpr int LATE = KR - KW > 0 ? KR - KW : 0;
        constexpr int Y0 = KW - 1 - i + NV0 + (i < LATE ? i : LATE);
        constexpr int younger = i < KW ? (Y0 < 15 ? Y0 : 15)
                                       : ((KR - 1 - i) < (KW - 1) ? (KR - 1 - i) : (KW - 1));
        lgkm_wait<kAsm, younger>(kf[i]);
        constexpr int ks = i / 2, kt = i % 2;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          s_new[rt][kt] = Elem<T>::mfma16(as_vec8<T>(kf[i]), qf[rt][ks], s_new[rt][kt]);
        if constexpr (i + KW < KR) kf[i + KW] = read_k(std::integral_constant<int, i + KW>{});
        if constexpr (HP) StaticFor<i * EA / KR, (i + 1) * EA / KR>::run(exp_pair);
      });
    } else if constexpr (HP) {
      StaticFor<0, NP>::run(exp_pair);
    }
    constexpr int EB = (HN && !KSPLIT) ? kExpA : NP;  // pairs done once stage A ends
    if constexpr (HP && !KSPLIT) {
      pb[0] = as_vec8<T>(w[0]);
      if constexpr (EB == NP) pb[1] = as_vec8<T>(w[1]);
    }

    // DS = 2: exchange with the partner wave: the partial S of its key tile
    // (s[rt][1]) for the partner's partial of ours, added to s[rt][0], and
    // the P words of the pending slice's own keys for the partner's, the
    // second half of the PV contraction.  Every wave of the workgroup takes
    // this path in the same calls, so the barriers are uniform.  A wave
    // writes its area only after a barrier that follows the partner's reads
    // of the previous contents: the sub-tile's barrier, or for the call of
    // the walk's last pending slice (no sub-tile), the barrier below.
    if constexpr ((HN || HP) && KSPLIT) {
      uint8_t* const mine = xbuf + wave * 4096;
      const uint8_t* const theirs = xbuf + (wave ^ (WAVES / 2)) * 4096;
      if constexpr (!HN) barrier_lds();
      if constexpr (HN) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) reinterpret_cast<f32x4*>(mine + 2048)[rt * 64 + lane] = s_new[rt][1];
      }
      if constexpr (HP)
        reinterpret_cast<u32x4*>(mine)[lane] = u32x4{w[0][0], w[0][1], w[1][0], w[1][1]};
      barrier_lds();
      if constexpr (HN) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const f32x4 v = reinterpret_cast<const f32x4*>(theirs + 2048)[rt * 64 + lane];
#pragma unroll
          for (int e = 0; e < 4; ++e) s_new[rt][0][e] += v[e];
        }
      }
      if constexpr (HP) {
        const u32x4 v = reinterpret_cast<const u32x4*>(theirs)[lane];
        w[0][2] = v[0];
        w[0][3] = v[1];
        w[1][2] = v[2];
        w[1][3] = v[3];
        pb[0] = as_vec8<T>(w[0]);
        pb[1] = as_vec8<T>(w[1]);
      }
    }

    // mask of the new slice (diagonal / partial slices only)
    if constexpr (HN && MASK) {
      // Element r of s[rt][kt] holds key 16kt + 4grp + r of the slice; it is
      // kept iff that key is < nkeys and (correction, or <= qpos - key0),
      // i.e. iff 16kt + r <= lim with one per-lane limit, so the tests
      // compare against immediates.  (DS = 2: only the own tile, whose keys
      // are 16*dhalf higher.)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int base = 4 * grp + (KSPLIT ? 16 * dhalf : 0);
        int lim = nw.nkeys - 1 - base;
        if (!nw.corr) lim = min(lim, qpos_abs[rt] - nw.key0 - base);
#pragma unroll
        for (int kt = 0; kt < (KSPLIT ? 1 : KT); ++kt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) s_new[rt][kt][r] = (16 * kt + r) <= lim ? s_new[rt][kt][r] : neg_inf();
        }
      }
    }

    // ---- stage B ----
    __builtin_amdgcn_s_setprio(1);
    // PV MFMAs of the pending slice with the row max of the new one spread
    // over them.  Each V^T fragment serves both row tiles: per batch, the
    // first row tile's MFMAs (over which the last exp pairs are spread),
    // then the second's.
    float mx[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) mx[rt] = neg_inf();
    constexpr int NM = KSPLIT ? 2 * RT : 4 * RT;  // max steps: one v_max3 per key pair
    auto max_step = [&](auto fc) {
      constexpr int f = decltype(fc)::value;
      constexpr int rt = f / (NM / RT), e = f % (NM / RT);
      constexpr int kt = e / 2, r0 = 2 * (e % 2);
      mx[rt] = fmaxf(fmaxf(mx[rt], s_new[rt][kt][r0]), s_new[rt][kt][r0 + 1]);
      asm volatile("" : "+v"(mx[rt]));
    };
    constexpr int PV_OPS = 2 * DT;  // PV MFMAs per slice
    if constexpr (HP) {
      lgkm_wait<kAsm, 0>(vb[0]);
      StaticFor<0, BATCHES>::run([&](auto bc) {
        constexpr int b = decltype(bc)::value;
        if constexpr (b + 1 < BATCHES) issue_v(va, std::integral_constant<int, b + 1>{}, vb[(b + 1) & 1], sp_c);
        constexpr int NQ = (DT - b * PER_BATCH) < PER_BATCH ? (DT - b * PER_BATCH) : PER_BATCH;
        StaticFor<0, 2 * PER_BATCH>::run([&](auto qc) {
          constexpr int j = decltype(qc)::value;
          constexpr int rt = j / PER_BATCH, q = j % PER_BATCH;
          if constexpr (q < NQ) {
            constexpr int dt = b * PER_BATCH + q;
            const u32x2(&r)[8] = vb[b & 1];
            const u32x4 av = {r[2 * q][0], r[2 * q][1], r[2 * q + 1][0], r[2 * q + 1][1]};
            o[dt][rt] = Elem<T>::mfma16(as_vec8<T>(av), pb[rt], o[dt][rt]);
            // the last exp pairs (the second row tile's) over the first
            // row tile's MFMAs of batch 0
            if constexpr (EB < NP && b == 0 && rt == 0) {
              StaticFor<EB + q * (NP - EB) / NQ, EB + (q + 1) * (NP - EB) / NQ>::run(exp_pair);
              if constexpr (q + 1 == NQ) pb[1] = as_vec8<T>(w[1]);
            }
            // the row max of the new slice, spread over the PV MFMAs (op:
            // this MFMA's index; every earlier batch is full)
            constexpr int op = b * 2 * PER_BATCH + rt * NQ + q;
            if constexpr (MAX) StaticFor<op * NM / PV_OPS, (op + 1) * NM / PV_OPS>::run(max_step);
          }
        });
        // the batch's MFMAs stay ahead of the wait for the next batch's
        // reads (otherwise the scheduler sinks them past it and the matrix
        // pipe idles while the reads land)
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (b + 1 < BATCHES) lgkm_wait<kAsm, 0>(vb[(b + 1) & 1]);
      });
      static_assert(PV_OPS == 2 * (BATCHES - 1) * PER_BATCH + 2 * (DT - (BATCHES - 1) * PER_BATCH),
                    "only the last batch is partial");
    } else if constexpr (MAX) {
      StaticFor<0, NM>::run(max_step);
    }

    // ---- stage C: reference max of the new slice ----
    // (the max over the four lanes of the row; DS = 2: then over the
    // partner's keys through LDS, whose previous read of this area was
    // consumed before the barrier of this sub-tile)
    auto row_max = [&](int rt) { return quad_max(mx[rt]); };
    float mrow[RT];
    if constexpr (MAX) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) mrow[rt] = row_max(rt);
      if constexpr (KSPLIT) {
        reinterpret_cast<f32x2*>(xbuf + wave * 4096 + 1024)[lane] = f32x2{mrow[0], mrow[1]};
        barrier_lds();
        const f32x2 v = reinterpret_cast<const f32x2*>(xbuf + (wave ^ (WAVES / 2)) * 4096 + 1024)[lane];
        mrow[0] = fmaxf(mrow[0], v[0]);
        mrow[1] = fmaxf(mrow[1], v[1]);
      }
    }
    if constexpr (MAX && MODE == 1) {
      // the first slice: O and l are still zero, no rescale
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        m_ref[rt] = fmaf(mrow[rt], c_pos, nw.corr ? a.shift : 0.f);
        neg_m[rt] = (m_ref[rt] == neg_inf()) ? 0.f : -m_ref[rt];
        m_thr[rt] = m_ref[rt] + kRescaleSlack;
      }
    }
    if constexpr (MAX && MODE == 2) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const float m_cand = fmaf(mrow[rt], c_pos, nw.corr ? a.shift : 0.f);  // -inf stays -inf (c_pos > 0)
        if (__ballot(m_cand > thr_of_ref(rt)) != 0ull) {
          const float m_new = fmaxf(m_ref[rt], m_cand);
          const float alpha = (m_new == neg_inf()) ? 1.f : __builtin_amdgcn_exp2f(m_ref[rt] - m_new);
          m_ref[rt] = m_new;
          if constexpr (kKeepRef) {
            neg_m[rt] = (m_ref[rt] == neg_inf()) ? 0.f : -m_ref[rt];
            m_thr[rt] = m_ref[rt] + kRescaleSlack;
          }
          l_run[rt] *= alpha;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) scale_in_place(o[dt][rt], alpha);
        }
      }
    }
    if constexpr (HN) p_pend = nw;
  };
  // The mask decision is taken before the call so that stages A and B stay
  // free of branches.
  auto process = [&](auto hn_c, auto hp_c, auto b_c, auto mode_c, const Slice& nw, auto sn_c, auto sp_c) {
    if constexpr (decltype(hn_c)::value) {
      if (needs_mask(nw)) process_m(hn_c, hp_c, b_c, std::true_type{}, mode_c, sn_c, sp_c, nw);
      else process_m(hn_c, hp_c, b_c, std::false_type{}, mode_c, sn_c, sp_c, nw);
    } else {
      process_m(hn_c, hp_c, b_c, std::false_type{}, mode_c, sn_c, sp_c, nw);
    }
  };

  // ---- pipelined walk: sub-tile `it` is multiplied from stage it % NST
  // while the fills of the next LA sub-tiles are in flight.  Fills past the
  // end load an empty sub-tile so every iteration issues the same number of
  // fills. ----
  using True = std::integral_constant<bool, true>;
  using False = std::integral_constant<bool, false>;
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  // cont_c: the walk continues an earlier walk's fixed reference.
  auto run_walk = [&](auto online_c, auto kind_c, auto cont_c) {
    constexpr bool ONLINE = decltype(online_c)::value;
    // (the reference-free pass computes no row max, not even for the first slice)
    using MFirst = std::integral_constant<int, ONLINE ? 2 : ((kFree || decltype(cont_c)::value) ? 0 : 1)>;
    using MRest = std::integral_constant<int, ONLINE ? 2 : 0>;
    const int count = walk_end - walk_it;  // sub-tiles of this walk
    Step pend[LA];
#pragma unroll
    for (int p = 0; p < LA; ++p) {
      pend[p] = next_step(kind_c);
      fill_step(pend[p], p, kind_c);
    }
    int cstage = 0;
    // One sub-tile (one slice).  The pending slice enters in s_buf[P] and
    // leaves in s_buf[1-P].
    auto do_step = [&](auto first_c, auto p_c) {
      constexpr bool FIRST = decltype(first_c)::value;
      constexpr int P = decltype(p_c)::value;
      using NewB = std::integral_constant<int, 1 - P>;
      fills_done();  // sub-tile it is in LDS; sub-tile it-2's stage is free
      const Step cur = pend[0];
#pragma unroll
      for (int p = 0; p < LA - 1; ++p) pend[p] = pend[p + 1];
      pend[LA - 1] = next_step(kind_c);
      const int fstage = cstage >= 2 ? cstage - 2 : cstage + NST - 2;
      fill_step(pend[LA - 1], fstage, kind_c);
      const Slice s0 = make_slice(cur, cstage, 0);
      if constexpr (FIRST) process(True{}, False{}, NewB{}, MFirst{}, s0, NoStage{}, NoStage{});
      else process(True{}, True{}, NewB{}, MRest{}, s0, NoStage{}, NoStage{});
      cstage = cstage == NST - 1 ? 0 : cstage + 1;
    };
    // The same with the ring stage known at compile time: sub-tile it is in
    // stage it % NST, so NST sub-tiles per iteration (a multiple of the
    // pending buffer's two).
    auto do_step_at = [&](auto first_c, auto p_c, auto st_c) {
      constexpr bool FIRST = decltype(first_c)::value;
      constexpr int P = decltype(p_c)::value;
      constexpr int ST = decltype(st_c)::value;
      using NewB = std::integral_constant<int, 1 - P>;
      using SP = std::integral_constant<int, (ST + NST - 1) % NST>;
      fills_done();
      const Step cur = pend[0];
#pragma unroll
      for (int p = 0; p < LA - 1; ++p) pend[p] = pend[p + 1];
      pend[LA - 1] = next_step(kind_c);
      fill_step(pend[LA - 1], (ST + LA) % NST, kind_c);
      const Slice s0 = make_slice(cur, ST, 0);
      if constexpr (FIRST) process(True{}, False{}, NewB{}, MFirst{}, s0, st_c, NoStage{});
      else process(True{}, True{}, NewB{}, MRest{}, s0, st_c, SP{});
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1 % NST>;
    using S2 = std::integral_constant<int, 2 % NST>;
    using S3 = std::integral_constant<int, 3 % NST>;
    // (exact walks only: in the correction and online walks the per-lane
    // addresses would stay live beside their own registers and spill)
    if constexpr (kImm && NST == 4 && decltype(kind_c)::value == 1) {
      if (count > 0) {
        do_step_at(True{}, P0{}, S0{});
        int it = 1;
        for (; it + 3 < count; it += 4) {
          do_step_at(False{}, P1{}, S1{});
          do_step_at(False{}, P0{}, S2{});
          do_step_at(False{}, P1{}, S3{});
          do_step_at(False{}, P0{}, S0{});
        }
        if (it < count) {
          do_step_at(False{}, P1{}, S1{});
          if (it + 1 < count) {
            do_step_at(False{}, P0{}, S2{});
            if (it + 2 < count) {
              do_step_at(False{}, P1{}, S3{});
              process(False{}, True{}, P1{}, MRest{}, p_pend, NoStage{}, S3{});
            } else {
              process(False{}, True{}, P0{}, MRest{}, p_pend, NoStage{}, S2{});
            }
          } else {
            process(False{}, True{}, P1{}, MRest{}, p_pend, NoStage{}, S1{});
          }
        } else {
          process(False{}, True{}, P0{}, MRest{}, p_pend, NoStage{}, S0{});
        }
      }
    } else if (count > 0) {
      do_step(True{}, P0{});  // the first sub-tile has no pending slice
      // the pending buffer alternates, so two sub-tiles per iteration
      int it = 1;
      for (; it + 1 < count; it += 2) {
        do_step(False{}, P1{});
        do_step(False{}, P0{});
      }
      if (it < count) {
        do_step(False{}, P1{});
        process(False{}, True{}, P1{}, MRest{}, p_pend, NoStage{}, NoStage{});  // pending in s_buf[0]
      } else {
        process(False{}, True{}, P0{}, MRest{}, p_pend, NoStage{}, NoStage{});  // pending in s_buf[1]
      }
    }
    // No fill may land in LDS after the walk ends.
    vm_wait<0>();
  };

  // First pass: no row's reference is ever updated, so the walk computes no
  // row max and never rescales O.  bfloat16: P = exp2(S) with no reference
  // (the logits in log2 units); float16: the reference is the max of the
  // row's first slice, P = exp2(s*c - m_ref).  P may then exceed 1 by any
  // factor: float32 sums and the 8-bit exponent of bfloat16 P hold it unless
  // the range is exceeded (float16 P past 2^16 is inf).  A valid row whose
  // sum leaves [2^-60, 2^64], or whose O holds an inf or NaN, sends the
  // workgroup through the walk again with the online reference and rescale
  // (kernel.py:287-310), where P <= 2^8.  The bound 2^64 keeps O finite for
  // |V| up to about 2^64; the finiteness test covers larger V.
  // Row sums: the four lanes of a row add their keys' sums (DS = 2: then the
  // two waves of a pair add theirs, in either order, so both hold the same
  // value).
  float l_tot[RT];
  auto row_sums = [&]() {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) l_tot[rt] = quad_sum(l_run[rt]);
    if constexpr (KSPLIT) {
      reinterpret_cast<f32x2*>(xbuf + wave * 4096 + 1024)[lane] = f32x2{l_tot[0], l_tot[1]};
      barrier_lds();
      const f32x2 v = reinterpret_cast<const f32x2*>(xbuf + (wave ^ (WAVES / 2)) * 4096 + 1024)[lane];
      l_tot[0] += v[0];
      l_tot[1] += v[1];
    }
  };
  if constexpr (kFree && CORR) {
    // exact steps, then the correction steps: in between, every weight so
    // far is scaled by 2^-shift = 1/block_k, which gives the pooled entries,
    // taken as exp2(S), their relative weight 2^shift (kernel.py:349-351);
    // O / l is unchanged by the common factor.  (A rescale inside the walk
    // would make the compiler move O between register ranges every slice.)
    // (every segment of a tile with correction steps takes the rescale,
    // so that their partials share one scale)
    walk_end = SEG ? min(s_hi, n_sel) : n_sel;
    // (the two walks are instantiated for their kinds of steps, except with
    // the D split, whose kernel measured 1 % slower with the second walk)
    using KindExact = std::integral_constant<int, KSPLIT ? 0 : 1>;
    using KindCorr = std::integral_constant<int, KSPLIT ? 0 : 2>;
    if (!SEG || walk_it < walk_end) run_walk(False{}, KindExact{}, False{});
    if (n_corr > 0) {
      __syncthreads();  // every wave is done with the ring before it is refilled
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        l_run[rt] *= a.inv_bk;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) scale_in_place(o[dt][rt], a.inv_bk);
      }
      walk_it = SEG ? max(s_lo, n_sel) : n_sel;
      walk_end = s_hi;
      if (!SEG || walk_it < walk_end) run_walk(False{}, KindCorr{}, False{});
    }
  } else if constexpr (CORR && !SEG && !KSPLIT) {
    // float16 with correction: the exact steps, then the correction steps,
    // whose slices keep the reference the first exact slice fixed.  (A
    // tile of the hook always selects a block, the largest energy passing
    // any alpha <= 1; a tile whose lists, given through the C ABI, select
    // none has no fixed reference and takes the online walk below.)
    walk_end = n_sel;
    run_walk(False{}, std::integral_constant<int, 1>{}, False{});
    if (n_corr > 0) {
      __syncthreads();  // every wave is done with the ring before it is refilled
      walk_it = n_sel;
      walk_end = s_hi;
      run_walk(False{}, std::integral_constant<int, 2>{}, True{});
    }
  } else {
    // (without correction every step is exact)
    run_walk(False{}, std::integral_constant<int, CORR ? 0 : 1>{}, False{});
  }
  row_sums();
  bool bad = false;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    bool fin = true;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) fin = fin && __builtin_isfinite(o[dt][rt][j]);
    }
    const float l = l_tot[rt];
    bad = bad || (row_valid[rt] && !(l >= 0x1p-60f && l <= 0x1p64f && fin));
  }
  if constexpr (CORR && !kFree && !SEG && !KSPLIT) bad = bad || n_sel == 0;  // (see the walks above)
  // Workgroup-wide decision through the last ring stage, which the second
  // walk refills only after its first barrier (the flags are read by then).
  int* const flags = reinterpret_cast<int*>(smem + (NST - 1) * GM::STAGE);
  __syncthreads();  // every wave is done with the ring
  const int wave_bad = __ballot(bad) != 0ull;  // every lane votes, then lane 0 stores
  if (lane == 0) flags[wave] = wave_bad;
  __syncthreads();
  int redo = 0;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) redo |= flags[w];
  if (redo) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt][rt] = f32x4{};
      m_ref[rt] = neg_inf();
      neg_m[rt] = 0.f;
      m_thr[rt] = neg_inf();
      l_run[rt] = 0.f;
    }
    p_pend = Slice{0, 0, 0, 0u};
    walk_it = s_lo;
    walk_end = s_hi;
    start_windows(s_lo);
    load_cids(max(s_lo - n_sel, 0) * BN);
    run_walk(True{}, std::integral_constant<int, 0>{}, False{});
    row_sums();
  }

  if constexpr (SEG) {
    // ---- a segment: unnormalised partials for merge_split_kernel ----
    // The partial is (O, l) * 2^m in the scale of exp2(logit): m = 0 for the
    // reference-free pass (log2(block_k) after its correction rescale), the
    // row's reference otherwise (a row that saw no key in its first slice
    // walked without one).
    const int item = (h * a.split_tiles + (t - (a.Nt - a.split_tiles))) * a.nchunk + chunk;
    const int64_t base = static_cast<int64_t>(item) * a.nseg + seg;
    float* const wo = a.ws_o + base * RW * D;
    float* const wml = a.ws_ml + base * RW * 2;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      if (!exists[rt]) continue;
      const int r = rwave * 32 + rt * 16 + l16;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        *reinterpret_cast<f32x4*>(wo + r * D + (dhalf * DT + dt) * 16 + grp * 4) = o[dt][rt];
      if (grp == 0 && dhalf == 0) {
        float m = m_ref[rt] == neg_inf() ? 0.f : m_ref[rt];
        if (kFree && !redo) m = (CORR && n_corr > 0) ? a.shift : 0.f;
        *reinterpret_cast<f32x2*>(wml + r * 2) = f32x2{m, l_tot[rt]};
      }
    }
    return;
  }

  // ---- normalise and store ----
  // O^T tile (dt, rt): the lane holds dims 16dt + 4grp + 0..3 of its row
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    if (!exists[rt] || pos[rt] >= a.out_rows) continue;
    const float inv = (row_valid[rt] && l_tot[rt] > 0.f) ? 1.f / l_tot[rt] : 0.f;
    uint16_t* orow = a.out + (static_cast<int64_t>(h) * a.G + g[rt]) * a.o_hs + pos[rt] * a.o_rs;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d0 = (dhalf * DT + dt) * 16 + grp * 4;
      u32x2 wv;
      wv[0] = pack2<T>(o[dt][rt][0] * inv, o[dt][rt][1] * inv);
      wv[1] = pack2<T>(o[dt][rt][2] * inv, o[dt][rt][3] * inv);
      *reinterpret_cast<u32x2*>(orow + d0) = wv;
    }
  }
}

// Merge of the split tiles' segments: row r of item (h, tile, chunk) is
// sum_s O_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), M the largest m_s of the
// segments with l_s > 0, written as the whole-tile kernel writes it (rows
// past the valid queries as zeros).  One thread per 4 dims of a row.
template <int D>
struct MergeShape {
  static constexpr int TPR = D / 4;         // threads per row
  static constexpr int ROWS = 256 / TPR;    // rows per workgroup
};
template <typename T, int D, int RW>
__global__ __launch_bounds__(256) void merge_split_kernel(AttnArgs a) {
  constexpr int TPR = MergeShape<D>::TPR, ROWS = MergeShape<D>::ROWS;
  constexpr int WPI = (RW + ROWS - 1) / ROWS;  // workgroups per item
  if (threadIdx.x >= TPR * ROWS) return;
  const int item = blockIdx.x / WPI;
  const int r = (blockIdx.x % WPI) * ROWS + threadIdx.x / TPR;
  const int d0 = (threadIdx.x % TPR) * 4;
  if (r >= RW) return;
  const int chunk = item % a.nchunk;
  const int ht = item / a.nchunk;
  const int h = ht / a.split_tiles;
  const int t = a.Nt - a.split_tiles + ht % a.split_tiles;
  const int prow = chunk * RW + r;
  if (prow >= a.G * a.tq) return;
  const int g = prow / a.tq;
  const int pos = t * a.tq + (prow - g * a.tq);
  if (pos >= a.out_rows) return;
  const int64_t base = static_cast<int64_t>(item) * a.nseg;
  float mx = neg_inf();
  for (int s = 0; s < a.nseg; ++s) {
    const f32x2 ml = *reinterpret_cast<const f32x2*>(a.ws_ml + ((base + s) * RW + r) * 2);
    if (ml[1] > 0.f) mx = fmaxf(mx, ml[0]);
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float l = 0.f;
  if (pos < a.Lq && mx != neg_inf()) {
    for (int s = 0; s < a.nseg; ++s) {
      const f32x2 ml = *reinterpret_cast<const f32x2*>(a.ws_ml + ((base + s) * RW + r) * 2);
      if (!(ml[1] > 0.f)) continue;
      const float w = __builtin_amdgcn_exp2f(ml[0] - mx);
      const f32x4 o = *reinterpret_cast<const f32x4*>(a.ws_o + ((base + s) * RW + r) * D + d0);
      acc += o * w;
      l += ml[1] * w;
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t* orow = a.out + (static_cast<int64_t>(h) * a.G + g) * a.o_hs + static_cast<int64_t>(pos) * a.o_rs;
  u32x2 wv;
  wv[0] = pack2<T>(acc[0] * inv, acc[1] * inv);
  wv[1] = pack2<T>(acc[2] * inv, acc[3] * inv);
  *reinterpret_cast<u32x2*>(orow + d0) = wv;
}

template <int WAVES, int DS>
constexpr int rows_per_wg() { return WAVES / DS * 32; }

// Split calls: the segments' launch, the whole tiles' launch, then the
// merge, in stream order.
template <typename T, int D, bool CORR, int WAVES, int NST, int DS = 1>
int launch_attn(AttnArgs a, hipStream_t stream) {
  constexpr int RW = rows_per_wg<WAVES, DS>();
  a.nchunk = (a.G * a.tq + RW - 1) / RW;
  const int64_t seg_wgs = static_cast<int64_t>(a.Hkv) * a.split_tiles * a.nchunk * a.nseg;
  const int64_t wgs = static_cast<int64_t>(a.Hkv) * (a.Nt - a.split_tiles) * a.nchunk;
  if (wgs > 0x7fffffffLL || seg_wgs > 0x7fffffffLL)
    return fail(FPV2_ERR_UNSUPPORTED, "sparse_attention: grid too large");
  if (seg_wgs > 0) {
    hipLaunchKernelGGL((sparse_attn_kernel<T, D, CORR, WAVES, NST, DS, true>),
                       dim3(static_cast<unsigned>(seg_wgs)), dim3(WAVES * 64), 0, stream, a);
    const int rc = check_launch("sparse_attention (segments)");
    if (rc) return rc;
  }
  if (wgs > 0) {
    hipLaunchKernelGGL((sparse_attn_kernel<T, D, CORR, WAVES, NST, DS, false>),
                       dim3(static_cast<unsigned>(wgs)), dim3(WAVES * 64), 0, stream, a);
    const int rc = check_launch("sparse_attention");
    if (rc) return rc;
  }
  if (seg_wgs == 0) return 0;
  constexpr int WPI = (RW + MergeShape<D>::ROWS - 1) / MergeShape<D>::ROWS;
  const int64_t mwgs = static_cast<int64_t>(a.Hkv) * a.split_tiles * a.nchunk * WPI;
  hipLaunchKernelGGL((merge_split_kernel<T, D, RW>), dim3(static_cast<unsigned>(mwgs)), dim3(256), 0,
                     stream, a);
  return check_launch("sparse_attention (merge)");
}

// Workgroup shape, 32-key sub-tiles in a 4-stage ring.  D <= 128: 4 waves
// (128 rows, 64 KiB, two workgroups per CU), tiles of more packed rows in
// 128-row chunks.  (An 8-wave shape over 64-key sub-tiles, sharing each fill
// between 256 rows, was measured no faster at 512-row tiles and up to 17 %
// slower at 256-row tiles.)  D = 256: 8 waves for 128 rows, two per 32-row
// group each owning half of D (DS = 2), 160 KiB.
template <typename T, int D, bool CORR>
int launch_shape(const AttnArgs& a, hipStream_t s) {
  if constexpr (D <= 128) {
    return launch_attn<T, D, CORR, 4, 4>(a, s);
  } else {
    return launch_attn<T, D, CORR, 8, 4, 2>(a, s);
  }
}

template <typename T>
int dispatch_attn(int64_t D, bool corr, const AttnArgs& a, hipStream_t s) {
  switch (D) {
    case 64: return corr ? launch_shape<T, 64, true>(a, s) : launch_shape<T, 64, false>(a, s);
    case 96: return corr ? launch_shape<T, 96, true>(a, s) : launch_shape<T, 96, false>(a, s);
    case 128: return corr ? launch_shape<T, 128, true>(a, s) : launch_shape<T, 128, false>(a, s);
    case 256: return corr ? launch_shape<T, 256, true>(a, s) : launch_shape<T, 256, false>(a, s);
    default:
      return fail(FPV2_ERR_UNSUPPORTED, "head dimension must be one of (64, 96, 128, 256)");
  }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace
}  // namespace fpv2

namespace fpv2 {
namespace {

// Validation of fpv2_sparse_attention's arguments and the kernel arguments
// they give; returns 0 or the failure status.
int attn_args(const void* q, const void* k, const void* v, const void* pooled_k,
              const void* pooled_v, const int32_t* selected_ids, const int32_t* selected_counts,
              const int32_t* pruned_ids, const int32_t* pruned_counts, void* out, int dtype,
              const fpv2_attn_params* p, AttnArgs* out_args) {
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
  if (p->pooled_head_stride < p->num_blocks * p->head_dim)
    return fail(FPV2_ERR_ARGUMENT, "sparse_attention: pooled_head_stride must be >= num_blocks*head_dim");
  if (p->pooled_head_stride % 8)
    return fail(FPV2_ERR_UNSUPPORTED, "sparse_attention: strides must be multiples of 8 elements");
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
  if (p->kv_heads * Nt * ((G * p->tile_q + 127) / 128) > 0x7fffffffLL ||
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
  a.c_scale = static_cast<float>(p->scale * 1.4426950408889634);
  a.shift = static_cast<float>(__builtin_log2(static_cast<double>(p->block_k)));
  a.inv_bk = static_cast<float>(1.0 / static_cast<double>(p->block_k));
  a.q_hs = p->q_head_stride;
  a.k_hs = p->k_head_stride;
  a.v_hs = p->v_head_stride;
  a.o_hs = p->o_head_stride;
  a.o_rs = p->o_row_stride;
  a.pooled_hs = p->pooled_head_stride;
  a.q_rs = static_cast<int>(p->q_row_stride);
  a.k_rs = static_cast<int>(p->k_row_stride);
  a.v_rs = static_cast<int>(p->v_row_stride);
  a.q_bytes = static_cast<uint32_t>(q_bytes);
  a.k_bytes = static_cast<uint32_t>(k_bytes);
  a.v_bytes = static_cast<uint32_t>(v_bytes);
  a.pooled_bytes = static_cast<uint32_t>(pooled_bytes);
  *out_args = a;
  return 0;
}

int dispatch(const AttnArgs& a, int dtype, const fpv2_attn_params* p, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool corr = p->mean_correction != 0;
  return dtype == FPV2_BF16 ? dispatch_attn<bf16_t>(p->head_dim, corr, a, s)
                            : dispatch_attn<f16_t>(p->head_dim, corr, a, s);
}

// Segments of the dense-tail split: the longest split tile is the last one,
// whose walk has at most nvis*subs exact steps (every block that starts at
// or before its last row) and ceil(Nb / 32) correction steps.
int64_t split_segments(const fpv2_attn_params* p, int64_t seg_steps) {
  const int64_t abs_last = p->offset + p->query_length - 1;
  const int64_t nvis = std::min<int64_t>(p->num_blocks, abs_last / p->block_k + 1);
  const int64_t subs = (p->block_k + 31) / 32;
  const int64_t steps = nvis * subs + (p->mean_correction ? (p->num_blocks + 31) / 32 : 0);
  return (steps + seg_steps - 1) / seg_steps;
}

constexpr int64_t kSplitRows = 128;  // packed query rows per workgroup, every shape

int64_t split_bytes(const fpv2_attn_params* p, int64_t split_tiles, int64_t seg_steps) {
  if (split_tiles == 0) return 0;
  const int64_t G = p->query_heads / p->kv_heads;
  const int64_t nchunk = (G * p->tile_q + kSplitRows - 1) / kSplitRows;
  const int64_t items = p->kv_heads * split_tiles * nchunk;
  return items * split_segments(p, seg_steps) * kSplitRows * (p->head_dim + 2) * 4;
}

}  // namespace
}  // namespace fpv2

extern "C" int fpv2_sparse_attention(const void* q, const void* k, const void* v,
                                     const void* pooled_k, const void* pooled_v,
                                     const int32_t* selected_ids, const int32_t* selected_counts,
                                     const int32_t* pruned_ids, const int32_t* pruned_counts,
                                     void* out, int dtype, const fpv2_attn_params* p,
                                     void* stream) {
  using namespace fpv2;
  AttnArgs a{};
  const int rc = attn_args(q, k, v, pooled_k, pooled_v, selected_ids, selected_counts, pruned_ids,
                           pruned_counts, out, dtype, p, &a);
  if (rc) return rc;
  return dispatch(a, dtype, p, stream);
}

extern "C" int64_t fpv2_sparse_attention_split_workspace_bytes(const fpv2_attn_params* p,
                                                               int64_t split_tiles,
                                                               int64_t seg_steps) {
  using namespace fpv2;
  if (!p || p->tile_q <= 0 || p->padded_query_length <= 0 || p->kv_heads <= 0 ||
      p->query_heads % p->kv_heads || p->block_k <= 0 || p->num_blocks <= 0 ||
      p->query_length <= 0)
    return fail(FPV2_ERR_ARGUMENT, "sparse_attention_split: invalid parameters");
  if (split_tiles < 0 || split_tiles > p->padded_query_length / p->tile_q || seg_steps < 1)
    return fail(FPV2_ERR_ARGUMENT, "sparse_attention_split: split_tiles must lie in [0, num_tiles] and seg_steps be positive");
  return split_bytes(p, split_tiles, seg_steps);
}

extern "C" int fpv2_sparse_attention_split(const void* q, const void* k, const void* v,
                                           const void* pooled_k, const void* pooled_v,
                                           const int32_t* selected_ids,
                                           const int32_t* selected_counts,
                                           const int32_t* pruned_ids, const int32_t* pruned_counts,
                                           void* out, int dtype, const fpv2_attn_params* p,
                                           int64_t split_tiles, int64_t seg_steps,
                                           void* workspace, int64_t workspace_bytes,
                                           void* stream) {
  using namespace fpv2;
  AttnArgs a{};
  const int rc = attn_args(q, k, v, pooled_k, pooled_v, selected_ids, selected_counts, pruned_ids,
                           pruned_counts, out, dtype, p, &a);
  if (rc) return rc;
  const int64_t need = fpv2_sparse_attention_split_workspace_bytes(p, split_tiles, seg_steps);
  if (need < 0) return static_cast<int>(need);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(FPV2_ERR_ARGUMENT, "sparse_attention_split: workspace of %lld bytes needed",
                static_cast<long long>(need));
  if (need > 0 && reinterpret_cast<uintptr_t>(workspace) % 16)
    return fail(FPV2_ERR_ARGUMENT, "sparse_attention_split: workspace must be 16-byte aligned");
  const int64_t nseg = split_segments(p, seg_steps);
  if (split_tiles * nseg * p->kv_heads > 0x7fffffffLL || seg_steps > 0x7fffffffLL)
    return fail(FPV2_ERR_UNSUPPORTED, "sparse_attention_split: too many segments");
  if (need > 0) {
    a.split_tiles = static_cast<int>(split_tiles);
    a.nseg = static_cast<int>(nseg);
    a.seg_steps = static_cast<int>(seg_steps);
    const int64_t G = p->query_heads / p->kv_heads;
    const int64_t items = p->kv_heads * split_tiles * ((G * p->tile_q + kSplitRows - 1) / kSplitRows);
    a.ws_o = static_cast<float*>(workspace);
    a.ws_ml = a.ws_o + items * nseg * kSplitRows * p->head_dim;
  }
  return dispatch(a, dtype, p, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free variant of fpv2_sparse_attention_split: the split's
// partials live in a file-scope device array, one copy per GPU, held until
// the process ends.  Its device address is taken once per device (with that
// device current) by hipGetSymbolAddress; host code never uses the array's
// name as an address.
namespace fpv2 {
namespace {

constexpr int64_t kScratchBytes = int64_t(64) << 20;  // FPV2_SPLIT_SCRATCH_BYTES
static_assert(kScratchBytes == FPV2_SPLIT_SCRATCH_BYTES, "header and source agree");
__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of the scratch array (set up on its first call).
int scratch_for_current_device(void** ptr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(FPV2_ERR_LAUNCH, "split_static: hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices) return fail(FPV2_ERR_UNSUPPORTED, "split_static: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(FPV2_ERR_LAUNCH, "split_static: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return 0;
}

}  // namespace
}  // namespace fpv2

extern "C" int fpv2_sparse_attention_split_static(const void* q, const void* k, const void* v,
                                                  const void* pooled_k, const void* pooled_v,
                                                  const int32_t* selected_ids,
                                                  const int32_t* selected_counts,
                                                  const int32_t* pruned_ids,
                                                  const int32_t* pruned_counts, void* out,
                                                  int dtype, const fpv2_attn_params* p,
                                                  int64_t split_tiles, int64_t seg_steps,
                                                  void* stream) {
  using namespace fpv2;
  const int64_t need = fpv2_sparse_attention_split_workspace_bytes(p, split_tiles, seg_steps);
  if (need < 0) return static_cast<int>(need);
  if (need > kScratchBytes)
    return fail(FPV2_ERR_UNSUPPORTED,
                "sparse_attention_split_static: the split needs %lld bytes of scratch; at most %lld",
                static_cast<long long>(need), static_cast<long long>(kScratchBytes));
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_for_current_device(&ws);
    if (rc) return rc;
  }
  return fpv2_sparse_attention_split(q, k, v, pooled_k, pooled_v, selected_ids, selected_counts,
                                     pruned_ids, pruned_counts, out, dtype, p, split_tiles,
                                     seg_steps, ws, need, stream);
}
