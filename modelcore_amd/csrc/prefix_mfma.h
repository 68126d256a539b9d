// Shared prompt prefix of a decode step on the matrix cores, as work the fused decode kernel runs
// before its streaming pass (decode_fused.hip): the queries of every row, all against keys
// [0, prefix) of row 0, which every row's keys below `prefix` are copies of.
//
// Semantics: modelcore/kernels/flash_attn.py:348-366 (T_new == 1, no window) restricted to the
// keys below the prefix; each job writes the unnormalised (o, m, l) of its key range per (row,
// query head), which the decode's merge pass combines with the row's own keys by log-sum-exp.
//
// Work split. A KV head's (row, query head) pairs -- rows x G of them, head fastest -- form
// groups of 32 (one wave's MFMA columns); a job owns one pair group, one KV head and one key
// range, and the workgroup's four waves (one per SIMD) split that range in four consecutive
// parts, each streaming its own 32-key tiles -- K straight into registers, V through its own
// double-buffered LDS, filled by DMA -- through v_mfma_f32_32x32x16_bf16:
//   S^T (keys x pairs) = K (keys x D) . Q^T (D x pairs)       A = K, B = Q, both in registers
//   O^T (D x pairs)   += V^T (D x keys) . P^T (keys x pairs)   A = V^T via ds_read_b64_tr_b16
// The transposed scores come out with one pair per lane (lane l: pair l % 32, keys 8 j + 4 (l /
// 32) + i), the layout the second product wants for its B operand; the 16 keys of a step are
// taken in that order, and the V^T fragment reads the same keys (two transpose reads of four
// rows). Online softmax per pair in fp32 (exp2 domain), the tile's maximum taken only when a
// pair's weights of the tile sum past 2^15, are not finite, or it has no maximum yet. No key of
// the prefix is masked: every decode query sits past it. The four waves' (o, m, l) are combined
// through LDS at the end, so the merge reads one partial per key range. Job ids place the pair
// groups of one (KV head, range) on one XCD (ids 8 apart), where they share its L2.
//
// The products' k index (the head dim) runs in any order common to both operands of S: fragment
// kd of lane half h holds dims 64 h + 8 kd .. + 7, so a lane's K of a tile is 128 contiguous
// bytes of its key's row (eight 16-byte loads) and its q likewise.
// V in LDS (per wave and buffer, 8 KiB): rows in natural order, 16-byte chunk c of row r at slot
// c ^ swz(r), under which the transpose reads (four consecutive rows, 32 bytes each per 16 lanes)
// use every bank. A job's LDS (65 KiB) and registers (at most 256) leave room for a streaming
// workgroup of the decode beside it on every compute unit.
#pragma once

#include <type_traits>

#include "kernels.h"

namespace mcamd {
namespace px {

constexpr int kD = 128;
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kKT = 32;              // keys per tile
constexpr int kTile = kKT * kD;      // elements of one K (or V) tile
constexpr int kMinKeys = 128;        // keys per range, at least
constexpr float kTileSumLimit = 32768.f;  // 2^15: a pair's weights of one tile sum to at most this
// LDS of a job: V tiles (two buffers per wave; the waves' o at the end), then their (m, l).
constexpr int kVBytes = kWaves * 2 * kTile * 2;
constexpr int kLdsBytes = kVBytes + 2 * kWaves * 32 * 4;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

struct Params {
  const uint16_t *q, *k_cache, *v_cache;  // q: (rows, H, D); keys and values of cache row 0
  float *part;  // slot ((row * n_units + unit) * n_split + range) of kDecodePartFloats floats
  int H, H_kv, G, n_pairs, n_pg, n_split, key_len, prefix, n_units, n_hc, T_max, jobs;
  float scale_log2;
};

// Key ranges: enough jobs to give each of `cus` compute units one, at most max_splits, and at
// least kMinKeys keys per range.
inline int splits(int64_t rows, int64_t n_head, int64_t n_kv_head, int64_t prefix, int cus,
                  int max_splits) {
  const int64_t G = n_head / n_kv_head;
  const int64_t per_split = n_kv_head * ((rows * G + 31) / 32);  // jobs per key range
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
__device__ __forceinline__ void ds_read_tr(bf16x4 &d, uint32_t addr) {
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(d) : "v"(addr), "i"(OFF));
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
  // Job id -> (KV head, key range, pair group).
  const int n_ks = P.H_kv * P.n_split;
  int ks, pg;
  if (n_ks % 8 == 0) {
    const int c = id >> 3;
    ks = (id & 7) + 8 * (c / P.n_pg);
    pg = c % P.n_pg;
  } else {
    ks = id / P.n_pg;
    pg = id - ks * P.n_pg;
  }
  const int kvh = ks / P.n_split;
  const int split = ks - kvh * P.n_split;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5;
  const int col = lane & 31;
  uint16_t *myV = reinterpret_cast<uint16_t *>(lds) + wave * 2 * kTile;
  float *sM = reinterpret_cast<float *>(lds + kVBytes);  // [kWaves][32]
  float *sL = sM + kWaves * 32;

  const int pr = pg * 32 + col;
  const bool live = pr < P.n_pairs;
  const int pp = live ? pr : P.n_pairs - 1;  // dead pairs compute on a live one
  const int row = pp / P.G;
  const int head = pp - row * P.G;

  // Q^T fragments: B[k = dim][n = pair], lane holds pair `col`, dims 64 h + 8 kd .. + 7. Loaded
  // as inline asm, ahead of every other load, and used only after the first tile's wait (which
  // then covers them): the compiler's own waits for tracked loads would also stall the first
  // tile on the second tile's DMAs.
  bf16x8 qf[8];
  {
    const uint16_t *qp = P.q + (int64_t(row) * P.H + int64_t(kvh) * P.G + head) * kD + 64 * h;
    asm volatile(
        "global_load_dwordx4 %0, %8, off\n"
        "global_load_dwordx4 %1, %8, off offset:16\n"
        "global_load_dwordx4 %2, %8, off offset:32\n"
        "global_load_dwordx4 %3, %8, off offset:48\n"
        "global_load_dwordx4 %4, %8, off offset:64\n"
        "global_load_dwordx4 %5, %8, off offset:80\n"
        "global_load_dwordx4 %6, %8, off offset:96\n"
        "global_load_dwordx4 %7, %8, off offset:112"
        : "=&v"(qf[0]), "=&v"(qf[1]), "=&v"(qf[2]), "=&v"(qf[3]), "=&v"(qf[4]), "=&v"(qf[5]),
          "=&v"(qf[6]), "=&v"(qf[7])
        : "v"(qp)
        : "memory");
  }

  // This wave's keys: part `wave` of the job's range [r_lo, r_hi) (never empty: at least
  // kMinKeys keys per range).
  const int r_lo = split * P.key_len;
  const int r_hi = min(P.prefix, r_lo + P.key_len);
  const int wl = (r_hi - r_lo + kWaves - 1) / kWaves;
  const int k_lo = r_lo + wave * wl;
  const int k_hi = min(r_hi, k_lo + wl);
  const int n_t = k_hi > k_lo ? (k_hi - k_lo + kKT - 1) / kKT : 0;

  // K/V of row 0's KV head as buffer resources: 32-bit byte offsets from the head's first
  // element, bounded by the last key of the cache.
  const uint32_t tok_bytes = uint32_t(P.H_kv) * kD * 2u;
  const uint32_t extent = uint32_t(P.T_max - 1) * tok_bytes + uint32_t(kD) * 2u;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(P.k_cache + int64_t(kvh) * kD), 0, int(extent), 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(P.v_cache + int64_t(kvh) * kD), 0, int(extent), 0x00020000);
  const uint32_t v_chunk = uint32_t((lane & 15) ^ (4 * ((lane >> 4) & 3)));
  // K of tile t into registers: fragment f of lane (key k0 + col, half h) = dims 64 h + 8 f ..
  // + 7 (keys past k_hi re-read k_hi - 1). Inline asm, like the q loads: the compiler counts
  // only its own loads, not the DMAs between them, and would wait for those too.
  const uint16_t *kbase = P.k_cache + int64_t(kvh) * kD + 64 * h;
  auto load_k = [&](bf16x8 (&kf)[8], int t) {
    const int key = min(k_lo + t * kKT + col, k_hi - 1);
    const uint16_t *kp = kbase + int64_t(key) * P.H_kv * kD;
    asm volatile(
        "global_load_dwordx4 %0, %8, off\n"
        "global_load_dwordx4 %1, %8, off offset:16\n"
        "global_load_dwordx4 %2, %8, off offset:32\n"
        "global_load_dwordx4 %3, %8, off offset:48\n"
        "global_load_dwordx4 %4, %8, off offset:64\n"
        "global_load_dwordx4 %5, %8, off offset:80\n"
        "global_load_dwordx4 %6, %8, off offset:96\n"
        "global_load_dwordx4 %7, %8, off offset:112"
        : "=&v"(kf[0]), "=&v"(kf[1]), "=&v"(kf[2]), "=&v"(kf[3]), "=&v"(kf[4]), "=&v"(kf[5]),
          "=&v"(kf[6]), "=&v"(kf[7])
        : "v"(kp)
        : "memory");
  };
  // V of tile t into buffer `buf`: eight blocks of four rows (chunks swizzled); keys past k_hi
  // re-read k_hi - 1.
  auto issue_v = [&](int t, int buf) {
    const int k0 = k_lo + t * kKT;
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      const uint32_t vkey = uint32_t(min(k0 + 4 * f + (lane >> 4), k_hi - 1));
      const uint32_t off = __umul24(vkey, tok_bytes) + ((v_chunk ^ uint32_t(f & 3)) << 4);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rv, (__attribute__((address_space(3))) void *)(myV + buf * kTile + f * 512), 16,
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
  uint32_t vofs[8];  // byte offsets of this lane's transpose reads for 16-key step 0
#pragma unroll
  for (int md = 0; md < 4; ++md) {
    const int r0 = 4 * h + tr_row, r1 = r0 + 8;
    const int cc = 32 * md + tr_col;
    vofs[md] = 2 * (r0 * kD + (((cc >> 3) ^ swz(r0)) << 3) + (cc & 7));
    vofs[4 + md] = 2 * (r1 * kD + (((cc >> 3) ^ swz(r1)) << 3) + (cc & 7));
  }

  // K one tile ahead in registers, V two tiles ahead in the LDS buffers. Load order: q, V(0),
  // K(0), V(1), then per tile t: K(t + 1) after the scores of t, V(t + 2) after its products.
  // At the top of tile t, K(t) and V(t) have landed once only the eight DMAs of V(t + 1) may be
  // pending (none when t is the last tile). The first wait also covers the q loads.
  auto wait_tile = [&](int t) {
    if (t + 1 < n_t)
      __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8)
    else
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    asm volatile("" ::: "memory");
  };
  bf16x8 kf[8];
  if (n_t > 0) {
    issue_v(0, 0);
    load_k(kf, 0);
  }
  if (n_t > 1) issue_v(1, 1);
  if (n_t == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // (no tile: the q loads)
  for (int t = 0; t < n_t; ++t) {
    const int buf = t & 1;
    wait_tile(t);
    // The registers the loads wrote are read only from here on.
    asm volatile(""
                 : "+v"(qf[0]), "+v"(qf[1]), "+v"(qf[2]), "+v"(qf[3]), "+v"(qf[4]), "+v"(qf[5]),
                   "+v"(qf[6]), "+v"(qf[7]), "+v"(kf[0]), "+v"(kf[1]), "+v"(kf[2]), "+v"(kf[3]),
                   "+v"(kf[4]), "+v"(kf[5]), "+v"(kf[6]), "+v"(kf[7]));
    const uint32_t vb = lds_addr(myV + buf * kTile);
    // S^T (32 keys x 32 pairs): s[4j + i] is key k0 + 8 j + 4 h + i of pair `col`.
    f32x16 s;
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = 0.f;
#pragma unroll
    for (int kd = 0; kd < 8; ++kd) s = mfma(kf[kd], qf[kd], s);
    if (t + 1 < n_t) load_k(kf, t + 1);
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
    // Every read of this buffer has completed (the wait above), so the DMA of tile t + 2 may
    // overwrite it.
    if (t + 2 < n_t) issue_v(t + 2, buf);
  }

  // Combine the four waves: each parks its (o, m, l) in its own (now idle) V tiles, then wave w
  // sums dims 32 w .. + 31 of all four, scaled to the common maximum, and writes them.
  const float lt = sum_halves(l);
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  float *red = reinterpret_cast<float *>(myV);  // 16 KiB: o[md][e] of lane at (md * 16 + e) * 64
#pragma unroll
  for (int md = 0; md < 4; ++md)
#pragma unroll
    for (int e = 0; e < 16; ++e) red[(md * 16 + e) * 64 + lane] = o[md][e];
  if (h == 0) {
    sM[wave * 32 + col] = m;
    sL[wave * 32 + col] = lt;
  }
  __syncthreads();
  float mw[kWaves], M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    mw[w] = sM[w * 32 + col];
    M = fmaxf(M, mw[w]);
  }
  float fw[kWaves], L = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    fw[w] = mw[w] == -INFINITY ? 0.f : exp2_or_zero(mw[w] - M);
    L += fw[w] * sL[w * 32 + col];
  }
  float acc[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const float *rw = reinterpret_cast<const float *>(lds) + w * 2 * kTile / 2 + wave * 16 * 64;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = fmaf(fw[w], rw[e * 64 + lane], acc[e]);
  }
  if (live) {
    // The unnormalised partial of (row, head) for this key range, in the decode unit's slot:
    // unit (row, KV-head group, query-head group), entry (KV head, query head) within it.
    const int unit = (kvh / kDecodeUnitKv) * P.n_hc + head / kDecodeUnitQ;
    const int entry = (kvh % kDecodeUnitKv) * kDecodeUnitQ + head % kDecodeUnitQ;
    float *slot =
        P.part + ((int64_t(row) * P.n_units + unit) * P.n_split + split) * kDecodePartFloats;
    float *po = slot + entry * kD + 32 * wave + 4 * h;  // dims 32 wave + 8 j + 4 h + i
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<float4 *>(po + 8 * j) =
          make_float4(acc[4 * j], acc[4 * j + 1], acc[4 * j + 2], acc[4 * j + 3]);
    if (wave == 0 && h == 0)
      *reinterpret_cast<float2 *>(slot + kDecodeUnitKv * kDecodeUnitQ * kD + 2 * entry) =
          make_float2(M, L);
  }
}

}  // namespace px
}  // namespace mcamd
