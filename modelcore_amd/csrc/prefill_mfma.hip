// Chunked-prefill attention against the cache prefix on the bf16 matrix cores (gfx950), for bf16
// caches with head_dim 128.
//
// Semantics: modelcore/kernels/flash_attn.py:226-244 (uniform rows: explicit causal + window mask
// with row offset Tk - Tq) and :362-364 (ragged rows). Query t of row b sits at
// p = cache_seqlens[b] + t and attends keys col <= p with p - col <= window when window >= 0;
// query head h reads KV head h / G; scale 1/sqrt(128). The append has already run, so the
// prefix includes the chunk itself.
//
// Work split. A workgroup owns one (row b, KV head) and 256 (position, query head) pairs of it:
// QT = 256 / G consecutive positions times the G query heads that share the KV head, head
// fastest (so one position's G heads are one contiguous run of q). Every K/V tile staged in LDS
// therefore serves the whole GQA group. Workgroup ids put the query tiles of one (b, KV head)
// 8 * k ids apart, so they land on the same XCD and share its L2.
//
// Eight waves, two per SIMD, in a ping-pong schedule (below): while one wave of a SIMD runs its
// products on the matrix core, its partner runs its softmax on the VALU. Each wave owns 32 pairs
// and computes, per tile of 64 keys, with v_mfma_f32_32x32x16_bf16 (16 + 16 instructions):
//   S^T (keys x pairs) = K (keys x D) . Q^T (D x pairs)       A = K from LDS, B = Q in registers
//   O^T (D x pairs)   += V^T (D x keys) . P^T (keys x pairs)   A = V^T via ds_read_tr16_b64
// Computing the transposed scores makes the score accumulators come out with one pair per lane
// (lane l holds pair l % 32, keys 8j + 4(l/32) + i), which is the layout the second product wants
// for its B operand: the eight consecutive accumulators of a 16-key step are that step's B
// fragment, once packed to bf16. The 16 keys of a step are taken in the order the accumulators
// hold them (4h..4h+3, then 8+4h..8+4h+3 for lane half h); the V^T fragment reads the same keys,
// as two LDS transpose reads of four rows each.
//
// Online softmax per pair in fp32 (exp2 domain): a tile's weights are made against the running
// maximum, and the tile's own maximum is taken (and O rescaled) only when a pair's weights of the
// tile sum past 2^15 or are not finite, or the pair has no maximum yet -- so most tiles skip both
// the maximum and the rescale, and weights stay below 2^15. Tiles entirely inside every pair's
// visible range skip the masking. The query fragments are multiplied by log2(e) / sqrt(128) once
// (rounded to bf16) and every score product starts from minus the running maximum instead of
// zero, so the scores leave the matrix core scaled and shifted and a weight is one exp2 (the
// per-score FMA that did both on the VALU is gone: +3.6%, 1110-1118 against 1072-1077 TFLOP/s).
//
// LDS: four buffers of one K and one V tile (64 keys x 256 bytes each), filled straight from
// HBM by buffer_load_dwordx4 ... lds (no registers involved) two tiles ahead of their first use;
// the buffer resource bounds every read to the (row, KV head)'s cache and keeps the per-lane
// address arithmetic in 32 bits. Each wave issues its four loads of a tile spread over its work
// of the slot, so no wave stalls on a full memory queue.
//  * K is stored fragment-major: 16 blocks of 1 KiB, block (mk, kd) holding exactly the A
//    fragment of keys 32 mk .. + 31 and dims 16 kd .. + 15 in lane order, so a wave reads a
//    fragment as one contiguous 1 KiB.
//  * V rows keep their natural order; 16-byte chunk c of row r sits at slot c ^ swz(r), under
//    which the transpose reads (4 consecutive rows, 32 bytes each per 16 lanes) use every bank.
// Both layouts were chosen by measuring the access patterns on MI355X (64 B/clk for row-strided
// 16-byte reads against ~100 B/clk contiguous; 134 B/clk for the swizzled transpose reads).
// In the matrix phase the LDS reads of the next 16-key step are issued (as inline asm, with
// explicit waits) while the products of the current one run, so the LDS streams under the
// MFMAs: pair by pair (one K fragment and one V^T fragment), each pair's reads waited for alone
// and the next step's reads of that pair issued right after (measured: +2.3% over issuing a
// step's twelve reads at once behind a wait for all of them).
//
// The shared prompt prefix of a decode step runs inside the fused decode kernel (prefix_mfma.h),
// built from the same fragments and layouts.
#include "kernels.h"

#include <cmath>
#include <type_traits>

namespace mcamd {
namespace {

constexpr int D = 128;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kPairs = 32 * kWaves;  // (position, head) pairs per workgroup
constexpr int KT = 64;               // keys per tile
constexpr int TILE = KT * D;         // elements of one K (or V) tile in LDS
constexpr float kTileSumLimit = 32768.f;  // 2^15: a pair's weights of one tile sum to at most this

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 lds_bf16x4 __attribute__((__vector_size__(4 * sizeof(__bf16))));

struct MfmaParams {
  const uint16_t *q, *k_cache, *v_cache;
  const int32_t *seqlens;
  const int32_t *rows, *cu;  // varlen prefill (optional): cache row and token range per sequence
  uint16_t *out;
  int T_new, H, H_kv, G, QT, T_max, window, n_bh;
  int64_t cache_b;
  float scale_log2;
};

__device__ __forceinline__ f32x16 mfma(const bf16x8 &a, const bf16x8 &b, const f32x16 &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Four consecutive LDS rows of one column, transposed into a lane: lane L of each 16-lane group
// passes the address of row L / 4, columns 4 (L % 4) .. + 3 of a 4 x 16 block and receives
// column L of it.
__device__ __forceinline__ bf16x4 lds_read_tr(const uint16_t *p) {
  auto lp = (__attribute__((address_space(3))) lds_bf16x4 *)(p);
  return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(lp));
}

// Swizzle of the 16-byte chunks of V row r (0..63): chunk c is stored at slot c ^ swz(r).
__device__ __forceinline__ int swz(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }

// LDS byte address of a pointer into shared memory.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return uint32_t(uintptr_t((const __attribute__((address_space(3))) void *)(p)));
}
// LDS reads issued as inline asm so they keep their place in the instruction stream. The
// compiler does not track them: every use of their results sits behind an explicit
// `s_waitcnt lgkmcnt(0)` asm that takes those results as operands (wait_all in the kernel).
template <int OFF>
__device__ __forceinline__ void ds_read_b128(bf16x8 &d, uint32_t addr) {
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(d) : "v"(addr), "i"(OFF));
}
template <int OFF>
__device__ __forceinline__ void ds_read_tr(bf16x4 &d, uint32_t addr) {
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(d) : "v"(addr), "i"(OFF));
}

// Waits until at most N LDS reads are pending; `r`, the result of an earlier one, is then ready.
template <int N>
__device__ __forceinline__ void lgkm_wait(bf16x8 &r) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(r) : "i"(N));
}

// Waits until at most N LDS reads are pending; a, b, c (results of earlier reads) are then ready.
template <int N>
__device__ __forceinline__ void lgkm_wait3(bf16x8 &a, bf16x4 &b, bf16x4 &c) {
  asm volatile("s_waitcnt lgkmcnt(%3)" : "+v"(a), "+v"(b), "+v"(c) : "i"(N));
}

// Across the two 32-lane halves of the wave (lane l with lane l ^ 32), on the VALU.
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float exp2_or_zero(float x) {
  return x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(x);
}

__global__ __launch_bounds__(kThreads, 1) void prefill_mfma_kernel(MfmaParams P) {
  __shared__ __attribute__((aligned(1024))) uint16_t sK[4][TILE];
  __shared__ __attribute__((aligned(1024))) uint16_t sV[4][TILE];

  const int bh = blockIdx.x % P.n_bh;
  const int qt = blockIdx.x / P.n_bh;
  const int b = bh / P.H_kv;  // sequence (a cache row, or one prompt of a varlen batch)
  const int kvh = bh - b * P.H_kv;
  const int q0 = qt * P.QT;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5;    // lane half
  const int col = lane & 31;  // this lane's pair within the wave's 32

  // Varlen: sequence b's queries are tokens [cu[b], cu[b + 1]) of q/out, its keys cache row
  // rows[b]; a query tile past the sequence's end has nothing to do (a whole workgroup).
  const int row = P.rows ? P.rows[b] : b;
  const int64_t tok0 = P.cu ? int64_t(P.cu[b]) : int64_t(b) * P.T_new;
  const int T_b = P.cu ? P.cu[b + 1] - P.cu[b] : P.T_new;
  if (q0 >= T_b) return;
  const int s0 = P.seqlens[row];
  const int q_end = min(q0 + P.QT, T_b);  // positions [q0, q_end) of the chunk
  const bool row_ok = s0 >= 0 && int64_t(s0) + T_b <= P.T_max;

  const int pr = wave * 32 + col;
  const bool live = pr < P.QT * P.G && q0 + pr / P.G < q_end;
  const int pos = live ? q0 + pr / P.G : q0;  // dead pairs compute on a live position
  const int head = live ? pr - (pr / P.G) * P.G : 0;
  uint16_t *out = P.out + ((tok0 + pos) * P.H + int64_t(kvh) * P.G + head) * D;
  if (!row_ok) {
    if (live)
      for (int d = h * 64; d < h * 64 + 64; ++d) out[d] = 0x7fc0;
    return;
  }

  // Q^T fragments: B[k = dim][n = pair], lane holds pair `col`, dims 16 kd + 8 h .. + 7, each
  // element multiplied by scale_log2 and rounded to bf16 once, so the products give scores in
  // log2 units with no per-score scaling.
  bf16x8 qf[8];
  {
    const uint16_t *qp = P.q + ((tok0 + pos) * P.H + int64_t(kvh) * P.G + head) * D + 8 * h;
#pragma unroll
    for (int kd = 0; kd < 8; ++kd) {
      const bf16x8 raw =
          __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(qp + 16 * kd));
      qf[kd] = __builtin_convertvector(__builtin_convertvector(raw, f32x8) * P.scale_log2, bf16x8);
    }
  }
  const int p_abs = s0 + pos;
  const int p_first = s0 + q0;
  const int p_last = s0 + q_end - 1;
  const int lo = P.window >= 0 ? max(0, p_first - P.window) : 0;
  const int hi = p_last;

  const int64_t tok = int64_t(P.H_kv) * D;
  const uint16_t *kbase = P.k_cache + int64_t(row) * P.cache_b + int64_t(kvh) * D;
  const uint16_t *vbase = P.v_cache + int64_t(row) * P.cache_b + int64_t(kvh) * D;

  // A tile takes 32 DMA instructions of 1 KiB (16 K fragments, 16 blocks of 4 V rows); wave w
  // issues K fragments 2w, 2w + 1 and V blocks 2w, 2w + 1. Keys past `hi` re-read key `hi` (they
  // are masked).
  // K/V of this (row, KV head) as buffer resources: 32-bit byte offsets from the head's first
  // element, bounded by the last key of the cache (out-of-range reads would return zero).
  const uint32_t tok_bytes = uint32_t(tok) * 2u;
  const uint32_t extent = uint32_t(P.T_max - 1) * tok_bytes + uint32_t(D) * 2u;
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc((void *)kbase, 0, int(extent), 0x00020000);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc((void *)vbase, 0, int(extent), 0x00020000);
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t k_lane_off = uint32_t(8 * h) * 2u;
  const uint32_t v_chunk = uint32_t((lane & 15) ^ (4 * ((lane >> 4) & 3)));
  // Part i (0..3) of this wave's share of a tile: K fragment 2w + i / 2 (i even) or V block
  // 2w + i / 2 (i odd).
  auto issue_part = [&](int k0, int buf, int i) {
    const int f = 2 * wave_s + (i >> 1);
    if ((i & 1) == 0) {
      const uint32_t kkey = uint32_t(min(k0 + 32 * (f >> 3) + col, hi));
      const uint32_t off = __umul24(kkey, tok_bytes) + uint32_t(16 * (f & 7)) * 2u + k_lane_off;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rk, (__attribute__((address_space(3))) void *)(&sK[buf][f * 512]), 16, int(off), 0, 0,
          0);
    } else {
      const uint32_t vkey = uint32_t(min(k0 + 4 * f + (lane >> 4), hi));  // row 4f + lane / 16
      const uint32_t off = __umul24(vkey, tok_bytes) + ((v_chunk ^ uint32_t(f & 3)) << 4);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rv, (__attribute__((address_space(3))) void *)(&sV[buf][f * 512]), 16, int(off), 0, 0,
          0);
    }
  };
  auto issue_tile = [&](int k0, int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) issue_part(k0, buf, i);
  };

  f32x16 o[4];
#pragma unroll
  for (int md = 0; md < 4; ++md)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[md][e] = 0.f;
  float m = -INFINITY;
  float l = 0.f;
  // The score products start from -m (the running maximum, 0 while the pair has none) in every
  // accumulator instead of zero, so a tile's scores arrive already shifted: the weights are
  // exp2 of them as they are. All sixteen accumulators of a lane belong to its one pair.
  f32x16 negm;
#pragma unroll
  for (int e = 0; e < 16; ++e) negm[e] = 0.f;

  const int L16 = lane & 15;
  const int tr_row = L16 >> 2;
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (L16 & 3);
  // Byte offsets of this lane's transpose reads in a V tile for 16-key step 0 (rows r0 = 4h +
  // tr_row and r0 + 8); step ks adds 4096 ks bytes, since the swizzle of rows 16 ks + r does not
  // depend on ks.
  uint32_t vofs[8];
#pragma unroll
  for (int md = 0; md < 4; ++md) {
    const int r0 = 4 * h + tr_row, r1 = r0 + 8;
    const int cc = 32 * md + tr_col;
    vofs[md] = 2 * (r0 * D + (((cc >> 3) ^ swz(r0)) << 3) + (cc & 7));
    vofs[4 + md] = 2 * (r1 * D + (((cc >> 3) ^ swz(r1)) << 3) + (cc & 7));
  }

  // Scores of one tile in log2 units less the running maximum: s[mk][4j + i] is key
  // k0 + 32 mk + 8 j + 4 h + i of pair `col`.
  auto scores = [&](f32x16 (&s)[2], const uint16_t *tK) {
#pragma unroll
    for (int kd = 0; kd < 8; ++kd)
#pragma unroll
      for (int mk = 0; mk < 2; ++mk) {
        const bf16x8 a = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4 *>(&tK[(mk * 8 + kd) * 512 + lane * 8]));
        s[mk] = mfma(a, qf[kd], kd == 0 ? negm : s[mk]);
      }
  };
  // Masks the keys the pair may not see (tiles that straddle the diagonal or the window edge).
  auto mask = [&](f32x16 (&s)[2], int k0) {
    const bool need_mask = (k0 + KT - 1 > p_first) || (P.window >= 0 && k0 < p_last - P.window);
    if (need_mask) {
#pragma unroll
      for (int mk = 0; mk < 2; ++mk)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = k0 + 32 * mk + 8 * (e >> 2) + 4 * h + (e & 3);
          const int dpos = p_abs - key;
          const bool ok = dpos >= 0 && (P.window < 0 || dpos <= P.window);
          if (!ok) s[mk][e] = -INFINITY;
        }
    }
  };
  // The tile's maximum score of the pair, in the units of `s` (log2, less the running maximum).
  auto tile_max = [&](const f32x16 (&s)[2]) {
    // Four independent chains, then across the two lane halves on the VALU.
    float m4[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int mk = 0; mk < 2; ++mk)
#pragma unroll
      for (int e = 0; e < 16; ++e) m4[e & 3] = fmaxf(m4[e & 3], s[mk][e]);
    return max_halves(fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3])));
  };
  // O^T += V^T . P^T for 16-key step ks, in the accumulators' key order.
  auto pv_step = [&](const bf16x8 &pk, int ks, const uint16_t *tV) {
    const int kb = 32 * (ks >> 1) + 16 * (ks & 1) + 4 * h;
    const int r0 = kb + tr_row, r1 = r0 + 8;
#pragma unroll
    for (int md = 0; md < 4; ++md) {
      const int cc = 32 * md + tr_col;  // column this lane addresses
      const bf16x4 lo4 = lds_read_tr(&tV[r0 * D + (((cc >> 3) ^ swz(r0)) << 3) + (cc & 7)]);
      const bf16x4 hi4 = lds_read_tr(&tV[r1 * D + (((cc >> 3) ^ swz(r1)) << 3) + (cc & 7)]);
      const bf16x8 a = __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
      o[md] = mfma(a, pk, o[md]);
    }
  };
  // Weights of 16-key step ks as the P^T fragment, and their sum: exp2 of the shifted scores,
  // less `shift` more when the maximum moved after the scores were made.
  auto sum8 = [](const f32x8 &pv) {
    return ((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7]));
  };
  auto weights = [&](const f32x16 (&s)[2], int ks, float &ts) {
    f32x8 pv;
#pragma unroll
    for (int e = 0; e < 8; ++e) pv[e] = __builtin_amdgcn_exp2f(s[ks >> 1][8 * (ks & 1) + e]);
    ts = sum8(pv);
    return __builtin_convertvector(pv, bf16x8);
  };
  auto weights_shifted = [&](const f32x16 (&s)[2], int ks, float shift, float &ts) {
    f32x8 pv;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      pv[e] = __builtin_amdgcn_exp2f(s[ks >> 1][8 * (ks & 1) + e] - shift);
    ts = sum8(pv);
    return __builtin_convertvector(pv, bf16x8);
  };

  // Ping-pong schedule over tiles of 64 keys, four LDS buffers. Each wave alternates a matrix
  // phase M(t) -- the scores of tile t + 1 and the P . V of tile t -- with a vector phase V(t) --
  // masks, maximum, rescale and weights of tile t. Waves 0-3 run one phase ahead of waves 4-7
  // (their SIMD partners), so in every slot one wave of each SIMD feeds the matrix core while
  // the other works the VALU. Slot 0 holds the first scores of group A, group B starts one slot
  // later and ends one slot later. Tile j (j >= 2) is fetched during slot 2 j - 4 into buffer
  // j % 4 and is read in slots 2 j .. 2 j + 3; tiles 0 and 1 are fetched before the loop.
  // A workgroup barrier opens every even slot 2 j (none at odd slots): it makes every wave's
  // DMAs of tile j visible (each wave waits for its own first) and ensures that every wave has
  // finished slot 2 j - 1, the last to read the buffer that tile j + 2 then takes. Within a pair
  // of slots the groups run free; a barrier at every slot, which only kept them in step,
  // measured 4.4% slower (1011-1013 against 1056-1058 TFLOP/s, two paired runs).
  const int n_tiles = (hi - lo) / KT + 1;
  const int lag = wave >= 4 ? 1 : 0;
  issue_tile(lo, 0);
  if (n_tiles > 1) issue_tile(lo + KT, 1);
  f32x16 sc[2];
  bf16x8 pk[4];
  for (int slot = 0; slot < 2 * n_tiles + 2; ++slot) {
    if ((slot & 1) == 0) {
      // Tile slot / 2 has landed once only the four DMAs of tile slot / 2 + 1 may be pending.
      if (slot / 2 + 1 < n_tiles)
        __builtin_amdgcn_s_waitcnt(0x0F74);  // vmcnt(4)
      else
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      // A bare barrier: __syncthreads' fence would make every wave wait for all its DMAs in
      // flight, the next tile's included, so that tile would have to land a pair of slots early.
      // Each wave's own vmcnt wait above has put its part of this tile in LDS, and every LDS
      // read of the buffer the next DMAs overwrite has been consumed before its wave got here.
      __builtin_amdgcn_s_barrier();
    }
    // Even slots fetch tile slot / 2 + 2 into buffer (slot / 2 + 2) % 4, whose previous tile was
    // last read in slot - 1; the four parts are spread over the slot's work.
    const int dma_tile = ((slot & 1) == 0 && slot / 2 + 2 < n_tiles) ? slot / 2 + 2 : -1;
    auto dma_part = [&](int i) {
      if (dma_tile >= 0) issue_part(lo + dma_tile * KT, dma_tile % 4, i);
    };
    const int ph = slot - lag;  // this wave's phase index
    if (ph < 0 || ph > 2 * n_tiles) {
      for (int i = 0; i < 4; ++i) dma_part(i);
      continue;
    }
    if (ph == 0) {
      for (int i = 0; i < 4; ++i) dma_part(i);
      scores(sc, sK[0]);
    } else if (ph & 1) {
      const int t = (ph - 1) / 2;  // V(t)
      mask(sc, lo + t * KT);
      // Weights against the running maximum the scores were shifted by (m_try); only when a
      // pair's weights of this tile sum past 2^15 (or are not finite), or the pair has no
      // maximum yet, is the tile's maximum taken, the accumulators rescaled, the weights made
      // again and the shift of later scores moved.
      const float m_try = m == -INFINITY ? 0.f : m;
      float ts[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) pk[ks] = weights(sc, ks, ts[ks]);
      float tl = (ts[0] + ts[1]) + (ts[2] + ts[3]);
      // The DMA parts after the weights (measured: ~1% faster than interleaved with them).
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) dma_part(ks);
      if (__builtin_amdgcn_ballot_w64(!(tl <= kTileSumLimit) || m == -INFINITY) != 0) {
        const float mx = tile_max(sc) + m_try;
        const float m_new = fmaxf(m, mx);
        const float alpha = m_new == -INFINITY ? 1.f : exp2_or_zero(m - m_new);
        l *= alpha;
#pragma unroll
        for (int md = 0; md < 4; ++md)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[md][e] *= alpha;
        m = m_new;
        const float m_use = m == -INFINITY ? 0.f : m;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) pk[ks] = weights_shifted(sc, ks, m_use - m_try, ts[ks]);
        tl = (ts[0] + ts[1]) + (ts[2] + ts[3]);
#pragma unroll
        for (int e = 0; e < 16; ++e) negm[e] = -m_use;
      }
      l += tl;
    } else {
      const int t = ph / 2 - 1;  // M(t)
      // The matrix phase at raised wave priority: when the matrix core frees, the SIMD issues
      // this wave's next product before its partner's VALU work (measured: +1.4-2.3% on the 16K
      // chunked prefill; the opposite preference costs 7%).
      __builtin_amdgcn_s_setprio(1);
      if (t + 1 < n_tiles) {
        // The two products interleaved; the twelve LDS reads of step ks + 1 (four K fragments,
        // four V^T fragments of two transpose reads) are issued before the eight products of
        // step ks, so the reads stream while the matrix core works.
        const uint32_t ka = lds_addr(&sK[(t + 1) % 4][lane * 8]);
        const uint32_t vb = lds_addr(sV[t % 4]);
        uint32_t va[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) va[i] = vb + vofs[i];
        bf16x8 kf[2][4];
        bf16x4 vf[2][4][2];
        // Pair i of step ks: K fragment i (keys 32 (i & 1) .., dims 16 (2 ks + i / 2) ..) and the
        // two transpose reads of V^T block i. Each pair's three reads are waited for alone, and
        // the next step's reads of the same pair are issued right after: LDS serves them spread
        // over the step instead of in one burst of twelve.
        auto issue_i = [&](auto ks_c, auto i_c, int buf) {
          constexpr int ks = decltype(ks_c)::value, i = decltype(i_c)::value;
          ds_read_b128<((i & 1) * 8 + 2 * ks + (i >> 1)) * 1024>(kf[buf][i], ka);
          ds_read_tr<4096 * ks>(vf[buf][i][0], va[i]);
          ds_read_tr<4096 * ks>(vf[buf][i][1], va[4 + i]);
        };
        auto wait_i = [&](auto n_c, auto i_c, int buf) {
          constexpr int n = decltype(n_c)::value, i = decltype(i_c)::value;
          lgkm_wait3<n>(kf[buf][i], vf[buf][i][0], vf[buf][i][1]);
        };
        auto pair = [&](auto ks_c, auto i_c) {
          constexpr int ks = decltype(ks_c)::value, i = decltype(i_c)::value;
          constexpr int cur = ks & 1;
          // Pending before the wait: this step's pairs i.. and the next step's pairs ..i - 1.
          wait_i(std::integral_constant<int, ks < 3 ? 9 : 3 * (3 - i)>{}, i_c, cur);
          if constexpr (ks < 3) issue_i(std::integral_constant<int, ks + 1>{}, i_c, cur ^ 1);
          constexpr int mk = i & 1, kd = 2 * ks + (i >> 1);
          sc[mk] = mfma(kf[cur][i], qf[kd], kd == 0 ? negm : sc[mk]);
          const bf16x8 a = __builtin_shufflevector(vf[cur][i][0], vf[cur][i][1], 0, 1, 2, 3, 4,
                                                   5, 6, 7);
          o[i] = mfma(a, pk[ks], o[i]);
          __builtin_amdgcn_sched_barrier(0);  // keep each pair's products right after its wait
        };
        auto step = [&](auto ks_c) {
          constexpr int ks = decltype(ks_c)::value;
          pair(ks_c, std::integral_constant<int, 0>{});
          pair(ks_c, std::integral_constant<int, 1>{});
          pair(ks_c, std::integral_constant<int, 2>{});
          pair(ks_c, std::integral_constant<int, 3>{});
          dma_part(ks);
        };
        auto issue = [&](auto ks_c, int buf) {
          issue_i(ks_c, std::integral_constant<int, 0>{}, buf);
          issue_i(ks_c, std::integral_constant<int, 1>{}, buf);
          issue_i(ks_c, std::integral_constant<int, 2>{}, buf);
          issue_i(ks_c, std::integral_constant<int, 3>{}, buf);
        };
        issue(std::integral_constant<int, 0>{}, 0);
        step(std::integral_constant<int, 0>{});
        step(std::integral_constant<int, 1>{});
        step(std::integral_constant<int, 2>{});
        step(std::integral_constant<int, 3>{});
      } else {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          pv_step(pk[ks], ks, sV[t % 4]);
          dma_part(ks);
        }
      }
      __builtin_amdgcn_s_setprio(0);
    }
  }

  // Normalise and write: o[md][4j + i] is dim 32 md + 8 j + 4 h + i of pair `col`.
  const float lt = sum_halves(l);
  const float inv = 1.f / lt;
  if (!live) return;
#pragma unroll
  for (int md = 0; md < 4; ++md)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x8 v8;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v8[i] = o[md][4 * j + i] * inv;
        v8[4 + i] = 0.f;
      }
      const bf16x8 w8 = __builtin_convertvector(v8, bf16x8);
      const bf16x4 w4 = __builtin_shufflevector(w8, w8, 0, 1, 2, 3);
      *reinterpret_cast<uint2 *>(out + 32 * md + 8 * j + 4 * h) = __builtin_bit_cast(uint2, w4);
    }
}

}  // namespace

bool prefill_mfma_geometry_ok(int64_t n_head, int64_t n_kv_head, int64_t t_max) {
  if (n_kv_head <= 0 || n_head < n_kv_head || t_max <= 0) return false;
  // Byte offsets within one (row, KV head) must fit the 32-bit buffer offsets.
  const int64_t extent = ((t_max - 1) * n_kv_head * D + D) * 2;
  return n_head / n_kv_head <= kPairs && n_kv_head < 65536 && extent < (int64_t(1) << 31);
}

bool prefill_mfma_supported(const AttnArgs &a) {
  return a.dtype == MCAMD_BF16 && a.head_dim == D &&
         prefill_mfma_geometry_ok(a.n_head, a.n_kv_head, a.t_max);
}

int launch_prefill_mfma(const AttnArgs &a) {
  MfmaParams P;
  P.q = static_cast<const uint16_t *>(a.q);
  P.k_cache = static_cast<const uint16_t *>(a.k_cache);
  P.v_cache = static_cast<const uint16_t *>(a.v_cache);
  P.seqlens = a.seqlens;
  P.rows = a.rows;
  P.cu = a.cu;
  P.out = static_cast<uint16_t *>(a.out);
  P.T_new = int(a.t_new);
  P.H = int(a.n_head);
  P.H_kv = int(a.n_kv_head);
  P.G = int(a.n_head / a.n_kv_head);
  P.QT = kPairs / P.G;
  P.T_max = int(a.t_max);
  P.window = int(a.window < 0 ? -1 : a.window);
  P.n_bh = int(a.batch * a.n_kv_head);
  P.cache_b = a.cache_batch_stride;
  P.scale_log2 = float(kLog2e / std::sqrt(double(D)));
  const int64_t n_qt = (a.t_new + P.QT - 1) / P.QT;
  const int64_t blocks = n_qt * P.n_bh;
  if (blocks > 0x7fffffff) return fail(MCAMD_EUNSUPPORTED, "prefill: grid too large");
  hipLaunchKernelGGL(prefill_mfma_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0,
                     a.stream, P);
  return launch_status("prefill_mfma");
}

}  // namespace mcamd

