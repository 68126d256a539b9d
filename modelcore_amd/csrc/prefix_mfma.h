// Shared prompt prefix of a decode step on the matrix cores, as work the fused decode kernel runs
// before its streaming pass (decode_fused.hip): the queries of every row, all against keys
// [0, prefix) of row 0, which every row's keys below `prefix` are copies of.
//
// Semantics: modelcore/kernels/flash_attn.py:348-366 (T_new == 1, no window) restricted to the
// keys below the prefix; each job writes the unnormalised (o, m, l) of its key range per (row,
// query head), which the decode's merge pass combines with the row's own keys by log-sum-exp.
//
// Work split. A KV head's (row, query head) pairs -- rows x G of them, head fastest -- form
// blocks of 64; a job owns one block, one KV head and one key range. Its four waves (one per
// SIMD) are two pair groups of 32 (one wave's MFMA columns) times two halves of the range: the
// two waves of a half share that half's 32-key K and V tiles, double-buffered in LDS and filled
// by DMA, and run them through v_mfma_f32_32x32x16_bf16:
//   S^T (keys x pairs) = K (keys x D) . Q^T (D x pairs)       A = K from LDS, B = Q in registers
//   O^T (D x pairs)   += V^T (D x keys) . P^T (keys x pairs)   A = V^T via ds_read_b64_tr_b16
// The transposed scores come out with one pair per lane (lane l: pair l % 32, keys 8 j + 4 (l /
// 32) + i), the layout the second product wants for its B operand; the 16 keys of a step are
// taken in that order, and the V^T fragment reads the same keys (two transpose reads of four
// rows). Online softmax per pair in fp32 (exp2 domain), the tile's maximum taken only when a
// pair's weights of the tile sum past 2^15, are not finite, or it has no maximum yet. No key of
// the prefix is masked: every decode query sits past it. The two halves' (o, m, l) of a pair
// group are combined through LDS at the end, so the merge reads one partial per key range. Job
// ids place the pair blocks of one (KV head, range) on one XCD (ids 8 apart), where they share
// its L2.
//
// LDS layout (per key half and buffer, 8 KiB each of K and V): the tile's rows in natural order,
// 16-byte chunk c of row r at slot c ^ swz(r). Each DMA then reads four whole rows (1 KiB
// contiguous: eight full cache lines), and both kinds of fragment read use every bank: a K
// fragment (sixteen consecutive rows per sixteen lanes, one chunk each) and a V^T transpose read
// (four consecutive rows, 32 bytes each per 16 lanes).
// A job's LDS (65 KiB) and registers (at most 256) leave room for a streaming workgroup of the
// decode beside it on every compute unit; the two share that CU's load path, so a job loads each
// K/V tile once for 64 pairs (half the bytes of one wave per 32 pairs).
#pragma once

#include "kernels.h"

namespace mcamd {
namespace px {

constexpr int kD = 128;
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kKT = 32;              // keys per tile
constexpr int kTile = kKT * kD;      // elements of one K (or V) tile
constexpr int kMinKeys = 128;        // keys per range, at least
constexpr int kPairsPerJob = 64;     // (row, query head) pairs of one KV head per job
constexpr float kTileSumLimit = 32768.f;  // 2^15: a pair's weights of one tile sum to at most this
// LDS of a job: two key halves x two buffers x (K tile + V tile), 64 KiB (the waves' o at the
// end), then the waves' (m, l).
constexpr int kTileBytes = 2 * 2 * 2 * kTile * 2;
constexpr int kLdsBytes = kTileBytes + 2 * kWaves * 32 * 4;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct Params {
  const uint16_t *q, *k_cache, *v_cache;  // q: (rows, H, D); keys and values of cache row 0
  char *part;  // slot ((row * n_units + unit) * n_split + range) of kPartSlotBytes
  int H, H_kv, G, n_pairs, n_pb, n_split, key_len, prefix, n_units, n_hc, T_max, jobs;
  float scale_log2;
};

// Key ranges: enough jobs to give each of `cus` compute units one, at most max_splits, and at
// least kMinKeys keys per range.
inline int splits(int64_t rows, int64_t n_head, int64_t n_kv_head, int64_t prefix, int cus,
                  int max_splits) {
  const int64_t G = n_head / n_kv_head;
  const int64_t per_split = n_kv_head * ((rows * G + kPairsPerJob - 1) / kPairsPerJob);
  const int64_t want = (int64_t(cus) + per_split - 1) / per_split;
  int64_t n = want < max_splits ? want : max_splits;
  if (n > prefix / kMinKeys) n = prefix / kMinKeys;
  return int(n < 1 ? 1 : n);
}

__device__ __forceinline__ f32x16 mfma(const bf16x8 &a, const bf16x8 &b, const f32x16 &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// Swizzle of the 16-byte chunks of V row r: chunk c is stored at slot c ^ swz(r).
__device__ __forceinline__ int swz(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return uint32_t(uintptr_t((const __attribute__((address_space(3))) void *)(p)));
}
// LDS transpose reads as inline asm: the compiler does not order them after pending DMAs (it
// would order every read of a tile after all of them, the next tile's included). Every result is
// used only behind an explicit `s_waitcnt lgkmcnt` that takes it as an operand.
template <int OFF>
__device__ __forceinline__ void ds_read_b128(bf16x8 &d, uint32_t addr) {
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(d) : "v"(addr), "i"(OFF));
}
template <int OFF>
__device__ __forceinline__ void ds_read_tr(bf16x4 &d, uint32_t addr) {
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(d) : "v"(addr), "i"(OFF));
}
template <int N>
__device__ __forceinline__ void lgkm_wait(bf16x8 &r) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(r) : "i"(N));
}
// Across the two 32-lane halves of the wave (lane l with lane l ^ 32).
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

// Job `id` (< P.jobs) of the prefix, run by all kThreads threads of the workgroup with `lds`
// pointing to kLdsBytes of shared memory (1 KiB aligned).
__device__ __forceinline__ void job(const Params &P, int id, unsigned char *lds) {
  // Job id -> (KV head, key range, block of kPairsPerJob pairs).
  const int n_ks = P.H_kv * P.n_split;
  int ks, pb;
  if (n_ks % 8 == 0) {
    const int c = id >> 3;
    ks = (id & 7) + 8 * (c / P.n_pb);
    pb = c % P.n_pb;
  } else {
    ks = id / P.n_pb;
    pb = id - ks * P.n_pb;
  }
  const int kvh = ks / P.n_split;
  const int split = ks - kvh * P.n_split;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave & 1;   // this wave's 32 pairs: the block's first or second
  const int half = wave >> 1; // this wave's half of the key range
  const int h = lane >> 5;
  const int col = lane & 31;
  // LDS: per key half, two buffers of one K tile and one V tile (both swizzled rows);
  // the two waves of a half (one per pair group) share them.
  uint16_t *sK = reinterpret_cast<uint16_t *>(lds) + half * 2 * kTile;
  uint16_t *sV = reinterpret_cast<uint16_t *>(lds) + (4 + half * 2) * kTile;
  float *sM = reinterpret_cast<float *>(lds + kTileBytes);  // [kWaves][32]
  float *sL = sM + kWaves * 32;

  const int pr = pb * kPairsPerJob + grp * 32 + col;
  const bool live = pr < P.n_pairs;
  const int pp = live ? pr : P.n_pairs - 1;  // dead pairs compute on a live one
  const int row = pp / P.G;
  const int head = pp - row * P.G;

  // Q^T fragments: B[k = dim][n = pair], lane holds pair `col`, dims 16 kd + 8 h .. + 7. Loaded
  // as inline asm, ahead of every DMA, and used only after the first tile's wait (which then
  // covers them): the compiler's own waits for tracked loads would also wait for DMAs.
  bf16x8 qf[8];
  {
    const uint16_t *qp = P.q + (int64_t(row) * P.H + int64_t(kvh) * P.G + head) * kD + 8 * h;
    asm volatile(
        "global_load_dwordx4 %0, %8, off\n"
        "global_load_dwordx4 %1, %8, off offset:32\n"
        "global_load_dwordx4 %2, %8, off offset:64\n"
        "global_load_dwordx4 %3, %8, off offset:96\n"
        "global_load_dwordx4 %4, %8, off offset:128\n"
        "global_load_dwordx4 %5, %8, off offset:160\n"
        "global_load_dwordx4 %6, %8, off offset:192\n"
        "global_load_dwordx4 %7, %8, off offset:224"
        : "=&v"(qf[0]), "=&v"(qf[1]), "=&v"(qf[2]), "=&v"(qf[3]), "=&v"(qf[4]), "=&v"(qf[5]),
          "=&v"(qf[6]), "=&v"(qf[7])
        : "v"(qp)
        : "memory");
  }

  // This wave's keys: half `half` of the job's range [r_lo, r_hi) (at least kMinKeys keys, so
  // both halves hold keys). Both halves take the same number of tiles (the barriers are the
  // workgroup's); keys past k_hi are masked.
  const int r_lo = split * P.key_len;
  const int r_hi = min(P.prefix, r_lo + P.key_len);
  const int hl = (r_hi - r_lo + 1) / 2;
  const int k_lo = r_lo + half * hl;
  const int k_hi = min(r_hi, k_lo + hl);
  const int n_t = (hl + kKT - 1) / kKT;

  // K/V of row 0's KV head as buffer resources: 32-bit byte offsets from the head's first
  // element, bounded by the last key of the cache.
  const uint32_t tok_bytes = uint32_t(P.H_kv) * kD * 2u;
  const uint32_t extent = uint32_t(P.T_max - 1) * tok_bytes + uint32_t(kD) * 2u;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(P.k_cache + int64_t(kvh) * kD), 0, int(extent), 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(P.v_cache + int64_t(kvh) * kD), 0, int(extent), 0x00020000);
  // A DMA lands lane i's 16 bytes at slot i % 16 of row i / 16 of its four rows, so lane i reads
  // the global chunk that belongs there: (i % 16) ^ swz(row).
  const uint32_t d_chunk = uint32_t((lane & 15) ^ (4 * ((lane >> 4) & 3)));
  // Tile t of this half into buffer t % 2: sixteen DMAs of 1 KiB, the half's wave of pair group
  // g issuing row blocks 4 g .. + 3 (rows 4 f .. 4 f + 3 of the tile) of K and of V; keys past
  // k_hi re-read k_hi - 1.
  auto issue_tile = [&](int t) {
    const int k0 = k_lo + t * kKT;
    const int buf = t & 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int f = 4 * grp + i;
      const uint32_t key = uint32_t(min(k0 + 4 * f + (lane >> 4), k_hi - 1));
      const uint32_t off = __umul24(key, tok_bytes) + ((d_chunk ^ uint32_t(f & 3)) << 4);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rk, (__attribute__((address_space(3))) void *)(sK + buf * kTile + f * 512), 16,
          int(off), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rv, (__attribute__((address_space(3))) void *)(sV + buf * kTile + f * 512), 16,
          int(off), 0, 0, 0);
    }
  };

  f32x16 o[4];
#pragma unroll
  for (int md = 0; md < 4; ++md)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[md][e] = 0.f;
  float m = -INFINITY;
  float l = 0.f;

  const int L16 = lane & 15;
  const int tr_row = L16 >> 2;
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (L16 & 3);
  // Byte offsets of this lane's K fragment reads: A[key][dim] of the scores' product, lane
  // (col, h) holding key col and dims 16 kd + 8 h .. + 7, i.e. chunk 2 kd + h of row col.
  uint32_t kofs[8];
#pragma unroll
  for (int kd = 0; kd < 8; ++kd)
    kofs[kd] = uint32_t(col * kD * 2 + (((2 * kd + h) ^ swz(col)) << 4));
  uint32_t vofs[8];  // byte offsets of this lane's transpose reads for 16-key step 0
#pragma unroll
  for (int md = 0; md < 4; ++md) {
    const int r0 = 4 * h + tr_row, r1 = r0 + 8;
    const int cc = 32 * md + tr_col;
    vofs[md] = 2 * (r0 * kD + (((cc >> 3) ^ swz(r0)) << 3) + (cc & 7));
    vofs[4 + md] = 2 * (r1 * kD + (((cc >> 3) ^ swz(r1)) << 3) + (cc & 7));
  }

  // One tile ahead. At the top of tile t, this wave's DMAs of tile t are its only ones pending
  // (the first wait also covers the q loads); the barrier then makes both waves' DMAs of the
  // half's tile t visible, and both have finished tile t - 1, whose buffer tile t + 1 then takes.
  // A bare barrier: a fence, even one for LDS alone, would wait for every DMA in flight.
  issue_tile(0);
  for (int t = 0; t < n_t; ++t) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __builtin_amdgcn_s_barrier();
    if (t + 1 < n_t) issue_tile(t + 1);
    asm volatile(""
                 : "+v"(qf[0]), "+v"(qf[1]), "+v"(qf[2]), "+v"(qf[3]), "+v"(qf[4]), "+v"(qf[5]),
                   "+v"(qf[6]), "+v"(qf[7]));
    const int buf = t & 1;
    const uint32_t kb = lds_addr(sK + buf * kTile);
    const uint32_t vb = lds_addr(sV + buf * kTile);
    bf16x8 kf[8];
#pragma unroll
    for (int kd = 0; kd < 8; ++kd) ds_read_b128<0>(kf[kd], kb + kofs[kd]);
    // S^T (32 keys x 32 pairs): s[4j + i] is key k0 + 8 j + 4 h + i of pair `col`.
    f32x16 s;
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = 0.f;
    lgkm_wait<7>(kf[0]);
    s = mfma(kf[0], qf[0], s);
    lgkm_wait<6>(kf[1]);
    s = mfma(kf[1], qf[1], s);
    lgkm_wait<5>(kf[2]);
    s = mfma(kf[2], qf[2], s);
    lgkm_wait<4>(kf[3]);
    s = mfma(kf[3], qf[3], s);
    lgkm_wait<3>(kf[4]);
    s = mfma(kf[4], qf[4], s);
    lgkm_wait<2>(kf[5]);
    s = mfma(kf[5], qf[5], s);
    lgkm_wait<1>(kf[6]);
    s = mfma(kf[6], qf[6], s);
    lgkm_wait<0>(kf[7]);
    s = mfma(kf[7], qf[7], s);
    // The V^T fragments of the first 16-key step, read while the softmax below runs (those of
    // the second step after it, while the first step's products run).
    bf16x4 vf[2][4][2];
    ds_read_tr<0>(vf[0][0][0], vb + vofs[0]);
    ds_read_tr<0>(vf[0][0][1], vb + vofs[4]);
    ds_read_tr<0>(vf[0][1][0], vb + vofs[1]);
    ds_read_tr<0>(vf[0][1][1], vb + vofs[5]);
    ds_read_tr<0>(vf[0][2][0], vb + vofs[2]);
    ds_read_tr<0>(vf[0][2][1], vb + vofs[6]);
    ds_read_tr<0>(vf[0][3][0], vb + vofs[3]);
    ds_read_tr<0>(vf[0][3][1], vb + vofs[7]);
    const int k0 = k_lo + t * kKT;
    if (k0 + kKT > k_hi) {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (k0 + 8 * (e >> 2) + 4 * h + (e & 3) >= k_hi) s[e] = -INFINITY;
    }
    // Weights against the running maximum; the tile's maximum is taken (and O rescaled) only
    // when a pair's weights of the tile sum past 2^15, are not finite, or it has no maximum yet.
    auto weights = [&](int step, float m_use, float &tl) {
      f32x8 pv;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        pv[e] = __builtin_amdgcn_exp2f(fmaf(s[8 * step + e], P.scale_log2, -m_use));
      tl += ((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7]));
      return __builtin_convertvector(pv, bf16x8);
    };
    float tl = 0.f;
    const float m_try = m == -INFINITY ? 0.f : m;
    bf16x8 pk0 = weights(0, m_try, tl), pk1 = weights(1, m_try, tl);
    if (__builtin_amdgcn_ballot_w64(!(tl <= kTileSumLimit) || m == -INFINITY) != 0) {
      float m4[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
      for (int e = 0; e < 16; ++e) m4[e & 3] = fmaxf(m4[e & 3], s[e]);
      const float mx =
          max_halves(fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]))) * P.scale_log2;
      const float m_new = fmaxf(m, mx);
      const float alpha = m_new == -INFINITY ? 1.f : exp2_or_zero(m - m_new);
      l *= alpha;
#pragma unroll
      for (int md = 0; md < 4; ++md)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[md][e] *= alpha;
      m = m_new;
      tl = 0.f;
      const float m_use = m == -INFINITY ? 0.f : m;
      pk0 = weights(0, m_use, tl);
      pk1 = weights(1, m_use, tl);
    }
    l += tl;
    ds_read_tr<16 * kD * 2>(vf[1][0][0], vb + vofs[0]);
    ds_read_tr<16 * kD * 2>(vf[1][0][1], vb + vofs[4]);
    ds_read_tr<16 * kD * 2>(vf[1][1][0], vb + vofs[1]);
    ds_read_tr<16 * kD * 2>(vf[1][1][1], vb + vofs[5]);
    ds_read_tr<16 * kD * 2>(vf[1][2][0], vb + vofs[2]);
    ds_read_tr<16 * kD * 2>(vf[1][2][1], vb + vofs[6]);
    ds_read_tr<16 * kD * 2>(vf[1][3][0], vb + vofs[3]);
    ds_read_tr<16 * kD * 2>(vf[1][3][1], vb + vofs[7]);
    // O^T += V^T . P^T over the tile's two 16-key steps, in the accumulators' key order.
    asm volatile("s_waitcnt lgkmcnt(8)"
                 : "+v"(vf[0][0][0]), "+v"(vf[0][0][1]), "+v"(vf[0][1][0]), "+v"(vf[0][1][1]),
                   "+v"(vf[0][2][0]), "+v"(vf[0][2][1]), "+v"(vf[0][3][0]), "+v"(vf[0][3][1])::
                     "memory");
#pragma unroll
    for (int md = 0; md < 4; ++md)
      o[md] = mfma(__builtin_shufflevector(vf[0][md][0], vf[0][md][1], 0, 1, 2, 3, 4, 5, 6, 7),
                   pk0, o[md]);
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(vf[1][0][0]), "+v"(vf[1][0][1]), "+v"(vf[1][1][0]), "+v"(vf[1][1][1]),
                   "+v"(vf[1][2][0]), "+v"(vf[1][2][1]), "+v"(vf[1][3][0]), "+v"(vf[1][3][1])::
                     "memory");
#pragma unroll
    for (int md = 0; md < 4; ++md)
      o[md] = mfma(__builtin_shufflevector(vf[1][md][0], vf[1][md][1], 0, 1, 2, 3, 4, 5, 6, 7),
                   pk1, o[md]);
  }

  // Combine the two halves of each pair group: every wave parks its (o, m, l) (after a barrier:
  // its partner may still read the tiles), then the wave of half x sums dims 64 x .. + 63 of
  // both, scaled to the common maximum, and writes them.
  const float lt = sum_halves(l);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  float *red = reinterpret_cast<float *>(lds) + wave * 4096;  // o[md][e] of lane at (md*16+e)*64
#pragma unroll
  for (int md = 0; md < 4; ++md)
#pragma unroll
    for (int e = 0; e < 16; ++e) red[(md * 16 + e) * 64 + lane] = o[md][e];
  if (h == 0) {
    sM[wave * 32 + col] = m;
    sL[wave * 32 + col] = lt;
  }
  __syncthreads();
  const int w0 = grp, w1 = grp + 2;  // the group's waves of halves 0 and 1
  const float m0 = sM[w0 * 32 + col], m1 = sM[w1 * 32 + col];
  const float M = fmaxf(m0, m1);
  const float f0 = m0 == -INFINITY ? 0.f : exp2_or_zero(m0 - M);
  const float f1 = m1 == -INFINITY ? 0.f : exp2_or_zero(m1 - M);
  const float L = f0 * sL[w0 * 32 + col] + f1 * sL[w1 * 32 + col];
  const float *r0 = reinterpret_cast<const float *>(lds) + w0 * 4096;
  const float *r1 = reinterpret_cast<const float *>(lds) + w1 * 4096;
  if (!live) return;
  // The unnormalised partial of (row, head) for this key range, in the decode unit's slot: unit
  // (row, KV-head group, query-head group), entry (KV head, query head) within it.
  const int unit = (kvh / kDecodeUnitKv) * P.n_hc + head / kDecodeUnitQ;
  const int entry = (kvh % kDecodeUnitKv) * kDecodeUnitQ + head % kDecodeUnitQ;
  char *slot =
      P.part + ((int64_t(row) * P.n_units + unit) * P.n_split + split) * kPartSlotBytes;
  // o[md][4 j + i] is dim 32 md + 8 j + 4 h + i; four of them rounded to bf16 make 8 bytes.
  uint16_t *po = reinterpret_cast<uint16_t *>(slot) + entry * kD + 4 * h;
#pragma unroll
  for (int mm = 0; mm < 2; ++mm) {
    const int md = 2 * half + mm;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4 a;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int idx = (md * 16 + 4 * j + i) * 64 + lane;
        a[i] = fmaf(f0, r0[idx], f1 * r1[idx]);
      }
      *reinterpret_cast<bf16x4 *>(po + 32 * md + 8 * j) = __builtin_convertvector(a, bf16x4);
    }
  }
  if (half == 0 && h == 0)
    *reinterpret_cast<float2 *>(slot + kPartSlotOBytes + 8 * entry) = make_float2(M, L);
}

}  // namespace px
}  // namespace mcamd
