// Single-token decode for bf16 caches with head_dim 128: append + attention in one balanced
// streaming pass over the cache, then a small merge pass.
//
// Semantics: modelcore/kernels/flash_attn.py:336-366 with T_new == 1 -- the new token's K/V land
// at p = cache_seqlens[b], and the query of row b attends keys [lo, p], lo = max(0, p - window)
// (window < 0: lo = 0); query head h reads KV head h / G; scale 1/sqrt(128).
//
// Layout facts the design rests on: the cache is (B, T_max, H_kv, 128) bf16, so one token's
// K (or V) for four consecutive KV heads is one contiguous 1 KiB run -- a whole wave64 load of
// 16 bytes per lane. On MI355X, streaming reads in such runs, with every CU given the same number
// of bytes, sustain ~6.5 TB/s; reads of one head's 256 bytes at a 1 KiB stride, or uneven work
// per CU, fall well short of that.
//
// Work split. A unit is (row b, group of four KV heads, group of up to four query heads per KV
// head). Laid end to end, the units form T = sum_b (n_b + C) * units slots (n_b = p_b - lo_b + 1
// keys, after C key-free lead slots that stand for the cost of starting a segment). The grid
// has a fixed number of workgroups (one per CU, a wave per SIMD), and workgroup g takes the slots
// [g*T/NG, (g+1)*T/NG): equal work for every CU whatever the row lengths. A workgroup's range is
// one or a few contiguous segments of units. Every workgroup derives T and its first row from
// cache_seqlens itself (a scan over the rows), so nothing is synchronised with the host.
//
// Inside a segment, lane (r, c) = (lane / 16, lane % 16) owns KV head 4*group + r and the 16
// bytes of dims c*8..c*8+7; a tile is four tokens (four loads each for K and V, the next tile's
// loads in flight while the current one is consumed).
//  * Scores: each lane forms partial dot products of its 8 dims with its KV head's 4 query heads
//    (v_dot2_f32_bf16 on packed bf16 pairs: 16 partials, 4 tokens x 4 heads), then a four-step
//    reduce-scatter over the 16 lanes of its row (DPP row_mirror, row_half_mirror, quad_perm)
//    leaves lane c with the complete score of token c/4 for head c%4.
//  * Softmax: a running maximum per head; a new maximum forces the rescale of the accumulators
//    only when it exceeds the current one by more than 2^8 (exp2 domain), so weights stay <= 256.
//  * Values: the 16 weights of a tile are broadcast inside the row (DPP row_newbcast) and packed
//    to bf16 pairs of consecutive tokens; the V rows of the same two tokens are interleaved with
//    v_perm_b32, so each v_dot2_f32_bf16 adds two tokens' contributions to one output dim.
//  * Output: a segment that covers its whole unit writes the normalised output; otherwise it
//    writes (o, m, l) for its 16 heads to the workspace (o rounded to bf16 once, m and l fp32:
//    half the bytes of fp32 partials, for ~0.5 us less per microbench call and 1.3% less per
//    mixed-window step, measured) -- segment j of unit u in bucket slot
//    u * 16 + j, segments past the sixteenth in an overflow slot (workgroup + unit, distinct per
//    segment since units advance with the workgroups) -- and the merge pass -- one wave per
//    (unit, query head), lane l owning dims 2l and 2l + 1 -- combines a unit's segments by
//    log-sum-exp. The workgroup holding a unit's first key records the unit's (first workgroup,
//    segment count), so the merge pass finds the partials without rebuilding the work split.
//  * Append: the segment that ends at p reads the new token from k/v instead of the cache and
//    its lanes store it into the cache at p (bit-exact copy; the first query-head group only).
//  * Shared prefix: when the caller states that every row's keys [0, S) are copies of row 0's
//    (rows replicated from one prompt), those keys come from row 0 for every row. A wide batch
//    with no window (at least 64 (row, query head) pairs per KV head, S >= 512) takes them on the
//    matrix cores first (prefix_mfma_kernel: every row's queries against row 0's keys, in key
//    ranges sized to fill the chip, one partial slot of each unit per range); this pass
//    then covers each row's keys from S on and writes partials even for a single segment, and
//    the merge folds the prefix partials in (sums in another order: within bf16 rounding of the
//    unshared call). Otherwise this pass reads the keys below S from row 0 itself: the same
//    values in the same order, the same results, with the rows' repeated reads of one row's
//    lines served by L2 and the memory-side cache instead of HBM.
#include "kernels.h"
#include "prefix_mfma.h"

#include <atomic>

#include <cmath>

namespace mcamd {
namespace {

constexpr int D = 128;
constexpr int GM = kDecodeUnitQ;      // query heads per KV head in one unit
constexpr int KG = kDecodeUnitKv;     // KV heads per unit (one per row of 16 lanes)
constexpr int kTokens = 4;            // tokens per tile
constexpr float kRescaleSlack = 8.f;  // log2 units
constexpr int kMaxGroups = 1024;      // 4-wave workgroups per launch, at most
#ifndef MCAMD_DECODE_GROUPS_PER_CU
#define MCAMD_DECODE_GROUPS_PER_CU 1
#endif
constexpr int kGroupsPerCU = MCAMD_DECODE_GROUPS_PER_CU;  // 1: one wave per SIMD
#ifndef MCAMD_DECODE_MIN_KEYS
#define MCAMD_DECODE_MIN_KEYS 72
#endif
constexpr int kMinKeysPerGroup = MCAMD_DECODE_MIN_KEYS;  // fewer workgroups when the job is small
#ifndef MCAMD_DECODE_RING
#define MCAMD_DECODE_RING 2
#endif
constexpr int kRing = MCAMD_DECODE_RING;  // tile buffers per wave (kRing - 1 tiles in flight)
#ifndef MCAMD_DECODE_WAVES
#define MCAMD_DECODE_WAVES 4
#endif
constexpr int NW = MCAMD_DECODE_WAVES;  // waves per workgroup: 4 (one per SIMD) or 8 (two)
static_assert(NW == 4 || NW == 8, "the four-row merge at a segment end takes 4 or 8 waves");
constexpr int kMergeSplit = NW / 4;          // waves per KV-head row in that merge
constexpr int kMergeDims = 128 / 16 / kMergeSplit;  // dims per lane in that merge (8 or 4)
#ifndef MCAMD_DECODE_SEG_COST
#define MCAMD_DECODE_SEG_COST 64
#endif
constexpr int kSegCost = MCAMD_DECODE_SEG_COST;  // key-free lead slots per unit (see unit_span)
// A partial slot: o[16][D] in bf16 (each fp32 sum rounded once, to nearest even), then
// (m, l)[16] in fp32 -- the same layout as the shared prefix's slots.
constexpr int kSlot = kPartSlotBytes;
constexpr int kSlotO = kPartSlotOBytes;
static_assert(kSlotO == KG * GM * D * 2 && kSlot == kSlotO + KG * GM * 8, "partial slot layout");
#ifndef MCAMD_DECODE_BUCKET
#define MCAMD_DECODE_BUCKET 16
#endif
// Partial slots per unit at addresses fixed by the unit alone (segment j of unit u in slot
// u * kBucket + j), so that the merge pass loads them in the same round trip as the unit's
// segment count; segments past kBucket go to an overflow area found through the descriptor.
constexpr int kBucket = MCAMD_DECODE_BUCKET;
#ifndef MCAMD_DECODE_SPEC
#define MCAMD_DECODE_SPEC 16
#endif
// Bucket slots the merge loads before the count is known, at most; a launch loads fewer (4 or 8)
// when its units average fewer segments (see launch_decode_fused).
constexpr int kSpec = MCAMD_DECODE_SPEC;
constexpr int64_t kTemporalLimit = int64_t(64) << 20;  // bytes of K/V: see launch_decode_fused
constexpr int64_t kPrefixMinKeys = 512;       // shorter shared prefixes stay in this pass
static_assert(kSpec <= kBucket, "speculative merge loads stay inside the unit's bucket");

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

struct FusedParams {
  const uint16_t *q, *k_new, *v_new;
  uint16_t *k_cache, *v_cache;
  const int32_t *seqlens;
  uint16_t *out;
  char *part;  // [B * n_units * kBucket] slots: segment j < kBucket of unit u at u * kBucket + j
  char *over;  // [kMaxGroups + B * n_units] slots: segments j >= kBucket, slot = group + unit
  int2 *desc;   // [B * n_units]: (first workgroup, segments) of each unit; (0, 0): no keys
  int32_t *adv_seqlens;  // the merge pass adds `advance` to every row's position (0: it does not)
  int advance;
  int shared;  // keys [0, shared) are read from row 0 for every row
  // Prefix on the matrix cores: this pass covers keys from lo_floor on, and the merge pass also
  // folds in n_pre partials per unit (slots unit * n_pre + j of `pre`, kPartSlotBytes each:
  // bf16 o, fp32 (m, l)) made for keys below it.
  int lo_floor;
  const char *pre;
  int n_pre;
  int B, H, H_kv, G, n_hc, n_kg, n_units, T_max, window, n_groups;
  int scan32;  // B <= 64 and every sum of row slot counts fits in 31 bits
  int64_t cache_b;
  float scale_log2;
};

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                         __builtin_bit_cast(bf16x2, b), c, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

// DPP controls (GFX9 encoding).
constexpr int kRowMirror = 0x140;
constexpr int kRowHalfMirror = 0x141;
constexpr int kQuadSwap3 = 0x1B;  // quad_perm [3,2,1,0]
constexpr int kQuadSwap1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kRowRor4 = 0x124;
constexpr int kRowRor8 = 0x128;
constexpr int kRowNewBcast = 0x150;  // + lane within the row
constexpr int kQuadBcast[4] = {0x00, 0x55, 0xAA, 0xFF};

template <int H>
__device__ __forceinline__ float quad_bcast(float x) {
  return dpp<kQuadBcast[H]>(x);
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ float exp2_or_zero(float x) {
  // exp2 of a difference whose left side may be -inf (masked key, or no key yet).
  return x == -INFINITY || x != x ? 0.f : fast_exp2(x);
}

// One reduce-scatter step over pairs of lanes (partner chosen by CTRL): a lane keeps the upper
// or lower half of v[0, 2N) according to `up`, adds the partner's copy of that half, and leaves
// the result in v[0, N).
template <int N, int CTRL>
__device__ __forceinline__ void rs_step(float (&v)[16], bool up) {
#pragma unroll
  for (int m = 0; m < N; ++m) {
    const float keep = up ? v[m + N] : v[m];
    const float send = up ? v[m] : v[m + N];
    v[m] = keep + dpp<CTRL>(send);
  }
}

struct Tile {
  uint4 k[kTokens], v[kTokens];
};

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// An empty use of a tile's registers: they stay allocated to it (and any load into them is
// waited for) up to this point, which comes after `anchor` is computed and before it is used.
__device__ __forceinline__ void keep_tile(const Tile &t, float &anchor) {
  asm volatile("" : "+v"(anchor)
               : "v"(__builtin_bit_cast(u32x4, t.k[0])), "v"(__builtin_bit_cast(u32x4, t.k[1])),
               "v"(__builtin_bit_cast(u32x4, t.k[2])), "v"(__builtin_bit_cast(u32x4, t.k[3])),
               "v"(__builtin_bit_cast(u32x4, t.v[0])), "v"(__builtin_bit_cast(u32x4, t.v[1])),
               "v"(__builtin_bit_cast(u32x4, t.v[2])), "v"(__builtin_bit_cast(u32x4, t.v[3])));
}

// Keys of a row at position pos (the range [lo, pos]), or 0 for a position outside the cache.
__device__ __forceinline__ int row_keys_at(const FusedParams &P, int pos, int &lo) {
  if (pos < 0 || pos >= P.T_max) {
    lo = 0;
    return 0;
  }
  lo = max(key_lo(pos, P.window), P.lo_floor);
  return max(pos - lo + 1, 0);
}
__device__ __forceinline__ int row_keys(const FusedParams &P, int b, int &lo) {
  return row_keys_at(P, P.seqlens[b], lo);
}

// Slots a unit of a row with nk keys takes in the work split: kSegCost lead slots that hold no
// keys, then its nk keys. The lead slots stand for what starting a segment costs a workgroup
// (refilling the load pipeline, the four-wave merge, the partial's write) in units of one key's
// streaming time, so a workgroup whose range holds the start of a unit gets fewer keys and
// finishes with the others.
__device__ __forceinline__ int unit_span(int nk) { return nk > 0 ? nk + kSegCost : 0; }

// Workgroup owning flattened slot x when T slots are shared out as [g*T/NG, (g+1)*T/NG).
__device__ __forceinline__ int group_of(int64_t x, int64_t T, int NG) {
  return int(((x + 1) * NG + T - 1) / T - 1);
}


__device__ __forceinline__ int64_t shfl_i64(int64_t v, int src) {
  const int lo = __shfl(int(uint64_t(v)), src, 64);
  const int hi = __shfl(int(uint64_t(v) >> 32), src, 64);
  return int64_t((uint64_t(uint32_t(hi)) << 32) | uint32_t(lo));
}

// Inclusive prefix sum over the 64 lanes in 32 bits, with DPP: shifts by 1, 2, 4, 8 within each
// row of 16 lanes, then the last lane of row r added to row r + 1 (row_bcast:15) and the last
// lane of row 1 to rows 2 and 3 (row_bcast:31); lanes with no source add 0.
__device__ __forceinline__ int scan_incl_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

__device__ __forceinline__ int64_t scan_incl_i64(int64_t v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t u = shfl_i64(v, max(lane - off, 0));
    if (lane >= off) v += u;
  }
  return v;
}

// Slots of rows [0, b_end) (every lane gets it).
__device__ int64_t slots_before(const FusedParams &P, int b_end, int lane) {
  int64_t total = 0;
  for (int b0 = 0; b0 < b_end; b0 += 64) {
    int lo;
    const int nk = b0 + lane < b_end ? row_keys(P, b0 + lane, lo) : 0;
    total += shfl_i64(scan_incl_i64(int64_t(unit_span(nk)) * P.n_units, lane), 63);
  }
  return total;
}

// Row holding slot x, and the first slot of that row.
__device__ void find_row(const FusedParams &P, int64_t x, int lane, int &b, int64_t &Pb) {
  int64_t carry = 0;
  b = -1;
  Pb = 0;
  for (int b0 = 0; b0 < P.B && b < 0; b0 += 64) {
    int lo;
    const int nk = b0 + lane < P.B ? row_keys(P, b0 + lane, lo) : 0;
    const int64_t tot = int64_t(unit_span(nk)) * P.n_units;
    const int64_t incl = scan_incl_i64(tot, lane);
    const uint64_t hit = __builtin_amdgcn_ballot_w64(carry + incl > x);
    if (hit) {
      const int l0 = __builtin_ctzll(hit);
      b = b0 + l0;
      Pb = carry + shfl_i64(incl - tot, l0);
    }
    carry += shfl_i64(incl, 63);
  }
}

// LDS image of one wave's accumulators at the end of a segment: o[row][head][D], m, l.
struct WaveAcc {
  float o[KG][GM][D];
  float m[KG][GM];
  float l[KG][GM];
};


// This workgroup's share of the slots: total T, active workgroups NG = min(n_groups, T), the
// range [start, end), and the row b holding `start` with Pb its first slot. With B <= 64 the
// rows' positions come in pos_lane (lane b holds row b's), read by the caller.
__device__ void locate(const FusedParams &P, int g, int lane, int pos_lane, int64_t &T, int &NG,
                       int64_t &start, int64_t &end, int &b, int64_t &Pb) {
  if (P.scan32) {
    int lo;
    const int nk = lane < P.B ? row_keys_at(P, pos_lane, lo) : 0;
    const int tot = unit_span(nk) * P.n_units;
    const int incl = scan_incl_i32(tot);
    T = __builtin_amdgcn_readlane(incl, 63);
    NG = int(min(int64_t(P.n_groups), T));
    if (g >= NG) return;
    start = int64_t(g) * T / NG;
    end = int64_t(g + 1) * T / NG;
    const uint64_t hit = __builtin_amdgcn_ballot_w64(incl > start);
    b = __builtin_ctzll(hit);
    Pb = __builtin_amdgcn_readlane(incl - tot, b);
    return;
  }
  if (P.B <= 64) {
    int lo;
    const int nk = lane < P.B ? row_keys_at(P, pos_lane, lo) : 0;
    const int64_t tot = int64_t(unit_span(nk)) * P.n_units;
    const int64_t incl = scan_incl_i64(tot, lane);
    T = shfl_i64(incl, 63);
    NG = int(min(int64_t(P.n_groups), T));
    if (g >= NG) return;
    start = int64_t(g) * T / NG;
    end = int64_t(g + 1) * T / NG;
    const uint64_t hit = __builtin_amdgcn_ballot_w64(incl > start);
    b = __builtin_ctzll(hit);
    Pb = shfl_i64(incl - tot, b);
    return;
  }
  T = slots_before(P, P.B, lane);
  NG = int(min(int64_t(P.n_groups), T));
  if (g >= NG) return;
  start = int64_t(g) * T / NG;
  end = int64_t(g + 1) * T / NG;
  find_row(P, start, lane, b, Pb);
}

// Work range of workgroup `id` of n: the dispatcher deals workgroup ids round-robin over the
// chip's 8 XCDs, so id's XCD is id % 8; ranges are given out XCD by XCD (XCD x takes a block of
// consecutive ranges), which keeps each XCD's reads within one part of the caches (measured on
// MI355X: decode microbench call 51.4 -> 51.0 us, mixed-window step 0.436 -> 0.428 ms).
__device__ __forceinline__ int xcd_major(int id, int n) {
  const int x = id % 8, i = id / 8;
  return x * (n / 8) + min(x, n % 8) + i;
}

// NT: K/V loads non-temporal (calls too large to stay in the memory-side cache) or with the
// default policy (small calls, whose K/V a KV-sharing layer may read again right after).
// The leading arguments repeat the fields of P that the first instructions need (the position
// scan, then the q and K/V addresses). The library is built with kernarg preloading (up to 16
// leading arguments, as many as fit the 14 free user SGPRs, stopping at the first aggregate):
// scalar arguments only, hence the copies. The scan then starts without waiting for a kernel-argument load from memory
// (measured: mixed-window step 0.394 -> 0.387 ms, decode call +0.3%, four paired runs).
// PX: workgroups n_groups and up run the shared prefix's matrix-core jobs instead (job
// blockIdx.x - n_groups), two workgroups to a compute unit, so that the jobs run beside the
// streaming workgroups.
template <bool NT, bool PX>
__device__ __forceinline__ void decode_fused_body(
    const int32_t *a_seqlens, const uint16_t *a_q, uint16_t *a_k_cache, uint16_t *a_v_cache,
    int a_B, int a_n_groups, int a_window, int a_lo_floor, int a_T_max, int a_n_units,
    FusedParams &P, const px::Params *X) {
  P.seqlens = a_seqlens;
  P.q = a_q;
  P.k_cache = a_k_cache;
  P.v_cache = a_v_cache;
  P.B = a_B;
  P.n_groups = a_n_groups;
  P.window = a_window;
  P.lo_floor = a_lo_floor;
  P.T_max = a_T_max;
  P.n_units = a_n_units;
  WaveAcc *s_acc;
  if constexpr (PX) {
    static_assert(NW == px::kWaves, "the prefix jobs take one wave per SIMD, four per workgroup");
    static_assert(sizeof(WaveAcc) * NW <= px::kLdsBytes, "the merge buffer fits the job's LDS");
    __shared__ __attribute__((aligned(1024))) unsigned char s_raw[px::kLdsBytes];
    if (int(blockIdx.x) >= P.n_groups) {
      px::job(*X, int(blockIdx.x) - P.n_groups, s_raw);
      return;
    }
    s_acc = reinterpret_cast<WaveAcc *>(s_raw);
  } else {
    __shared__ WaveAcc s_acc_own[NW];
    s_acc = s_acc_own;
  }
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;  // wave within the workgroup
  const int g = xcd_major(int(blockIdx.x), P.n_groups);
  const int r = lane >> 4;  // KV head within the unit's group of four
  const int c = lane & 15;  // 16-byte column of the head row

  // With at most 64 rows, the positions are read once, first thing (lane b holds row b's): the
  // check of rows outside the cache, the work split and each segment's row take them from here,
  // so the work split does not wait for a second read of cache_seqlens.
  const bool few_rows = P.B <= 64;
  const int pos_lane = few_rows && lane < P.B ? P.seqlens[lane] : 0;
  auto row_pos = [&](int row) {
    return few_rows ? __builtin_amdgcn_readlane(pos_lane, row) : P.seqlens[row];
  };
  // Rows outside the cache: NaN output and a descriptor of no segments for each of their units
  // (so the merge pass need not read cache_seqlens), written by workgroup b % n_groups.
  for (int b = g; b < P.B; b += P.n_groups) {
    int lo;
    if (row_keys_at(P, row_pos(b), lo) == 0) {
      for (int i = threadIdx.x; i < P.H * D; i += 64 * NW) P.out[int64_t(b) * P.H * D + i] = 0x7fc0;
      for (int u = threadIdx.x; u < P.n_units; u += 64 * NW)
        P.desc[int64_t(b) * P.n_units + u] = make_int2(0, 0);
    }
  }
  // NG <= T active workgroups: every range [g*T/NG, (g+1)*T/NG) is then non-empty, so the
  // workgroups holding a unit's keys are exactly those from its first key's owner to its last
  // key's (a range of lead slots alone holds no key of the unit and writes nothing for it).
  int64_t T, start = 0, end = 0, Pb = 0;
  int NG, b = 0;
  locate(P, g, lane, pos_lane, T, NG, start, end, b, Pb);
  if (g >= NG) return;

  const bool fuse_new = P.k_new != nullptr;
  const int64_t tok_stride = int64_t(P.H_kv) * D;
  int64_t x = start;
  while (x < end) {
    int lo;
    const int nk = row_keys_at(P, row_pos(b), lo);
    const int span = unit_span(nk);
    const int pos = lo + nk - 1;
    const int64_t off = x - Pb;
    const int unit = int(off / span);
    const int lead = int(off - int64_t(unit) * span);
    if (lead < kSegCost) {  // the unit's lead slots: no keys to stream
      x += kSegCost - lead;
      continue;
    }
    const int t_rel = lead - kSegCost;
    const int seg = int(min(end - x, int64_t(nk - t_rel)));
    const int ts = lo + t_rel;  // first key of the segment
    const int last = ts + seg - 1;

    const int kg = unit / P.n_hc;
    const int hc = unit - kg * P.n_hc;
    const int kvh_raw = kg * KG + r;
    const bool row_live = kvh_raw < P.H_kv;
    const int kvh = row_live ? kvh_raw : P.H_kv - 1;  // idle rows re-read a live head
    const int h0 = kvh * P.G + hc * GM;
    const int gcount = row_live ? min(GM, P.G - hc * GM) : 0;
    const bool append_here = fuse_new && hc == 0 && row_live;

    // Query heads of this lane's KV head, packed bf16 pairs of its 8 dims (zero past gcount).
    uint4 qv[GM];
#pragma unroll
    for (int h = 0; h < GM; ++h)
      qv[h] = h < gcount ? *reinterpret_cast<const uint4 *>(P.q + (int64_t(b) * P.H + h0 + h) * D + c * 8)
                         : make_uint4(0, 0, 0, 0);

    const uint16_t *kbase = P.k_cache + int64_t(b) * P.cache_b + int64_t(kvh) * D + c * 8;
    const uint16_t *vbase = P.v_cache + int64_t(b) * P.cache_b + int64_t(kvh) * D + c * 8;
    // Row 0's copy of the keys every row shares (the same bytes as the row's own).
    const uint16_t *kbase0 = P.k_cache + int64_t(kvh) * D + c * 8;
    const uint16_t *vbase0 = P.v_cache + int64_t(kvh) * D + c * 8;
    const int64_t new_off = (int64_t(b) * P.H_kv + kvh) * D + c * 8;

    // Loads are unconditional (keys past the segment re-read its last key and are masked), so
    // the prefetch of the next tile is straight-line code and stays in flight.
    auto load_tile = [&](Tile &Tl, int tile) {
#pragma unroll
      for (int j = 0; j < kTokens; ++j) {
        const int t = min(ts + tile * kTokens + j, last);
        const bool is_new = fuse_new && t == pos;
        const bool shared = t < P.shared;
        const uint16_t *kp =
            is_new ? P.k_new + new_off : (shared ? kbase0 : kbase) + int64_t(t) * tok_stride;
        const uint16_t *vp =
            is_new ? P.v_new + new_off : (shared ? vbase0 : vbase) + int64_t(t) * tok_stride;
        if constexpr (NT) {
          Tl.k[j] = load_stream(kp);
          Tl.v[j] = load_stream(vp);
        } else {
          Tl.k[j] = *reinterpret_cast<const uint4 *>(kp);
          Tl.v[j] = *reinterpret_cast<const uint4 *>(vp);
        }
      }
    };

    float m = -INFINITY;  // running max (exp2 domain) of this lane's head c%4
    float l = 0.f;        // this lane's own sum of weights
    float o[GM][8];
#pragma unroll
    for (int h = 0; h < GM; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[h][e] = 0.f;

    auto process = [&](const Tile &Tl, int tile) {
      if (append_here && pos <= last) {
#pragma unroll
        for (int j = 0; j < kTokens; ++j) {
          if (ts + tile * kTokens + j == pos) {
            const int64_t at = int64_t(b) * P.cache_b + int64_t(pos) * tok_stride + int64_t(kvh) * D + c * 8;
            *reinterpret_cast<uint4 *>(P.k_cache + at) = Tl.k[j];
            *reinterpret_cast<uint4 *>(P.v_cache + at) = Tl.v[j];
          }
        }
      }
      // Partial scores xs[4j + h] over this lane's 8 dims.
      float xs[16];
#pragma unroll
      for (int j = 0; j < kTokens; ++j) {
#pragma unroll
        for (int h = 0; h < GM; ++h) {
          float a = dot2(Tl.k[j].x, qv[h].x, 0.f);
          a = dot2(Tl.k[j].y, qv[h].y, a);
          a = dot2(Tl.k[j].z, qv[h].z, a);
          a = dot2(Tl.k[j].w, qv[h].w, a);
          xs[4 * j + h] = a;
        }
      }
      // Reduce-scatter over the row: lane c ends with value index c = 4j + h.
      rs_step<8, kRowMirror>(xs, c >= 8);
      rs_step<4, kRowHalfMirror>(xs, (c & 7) >= 4);
      rs_step<2, kQuadSwap3>(xs, (c & 3) >= 2);
      rs_step<1, kQuadSwap1>(xs, (c & 1) != 0);
      const int tt = tile * kTokens + (c >> 2);
      const float sc = tt < seg ? xs[0] * P.scale_log2 : -INFINITY;

      // Maximum per head over the tile: lanes c, c+4, c+8, c+12 share head c%4.
      float mx = fmaxf(sc, dpp<kRowRor4>(sc));
      mx = fmaxf(mx, dpp<kRowRor8>(mx));
      if (__builtin_amdgcn_ballot_w64(mx > m + kRescaleSlack) != 0) {
        const float m_new = fmaxf(m, mx);
        const float alpha = m_new == -INFINITY ? 1.f : exp2_or_zero(m - m_new);
        l *= alpha;
        const float a0 = quad_bcast<0>(alpha), a1 = quad_bcast<1>(alpha);
        const float a2 = quad_bcast<2>(alpha), a3 = quad_bcast<3>(alpha);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          o[0][e] *= a0;
          o[1][e] *= a1;
          o[2][e] *= a2;
          o[3][e] *= a3;
        }
        m = m_new;
      }
      const float p = sc == -INFINITY ? 0.f : fast_exp2(sc - m);
      l += p;

      // Weights of the tile's 4 tokens x 4 heads, packed as (token 2i, token 2i+1) pairs.
      uint32_t pp[GM][2];
      pp[0][0] = pack_bf16(dpp<kRowNewBcast + 0>(p), dpp<kRowNewBcast + 4>(p));
      pp[1][0] = pack_bf16(dpp<kRowNewBcast + 1>(p), dpp<kRowNewBcast + 5>(p));
      pp[2][0] = pack_bf16(dpp<kRowNewBcast + 2>(p), dpp<kRowNewBcast + 6>(p));
      pp[3][0] = pack_bf16(dpp<kRowNewBcast + 3>(p), dpp<kRowNewBcast + 7>(p));
      pp[0][1] = pack_bf16(dpp<kRowNewBcast + 8>(p), dpp<kRowNewBcast + 12>(p));
      pp[1][1] = pack_bf16(dpp<kRowNewBcast + 9>(p), dpp<kRowNewBcast + 13>(p));
      pp[2][1] = pack_bf16(dpp<kRowNewBcast + 10>(p), dpp<kRowNewBcast + 14>(p));
      pp[3][1] = pack_bf16(dpp<kRowNewBcast + 11>(p), dpp<kRowNewBcast + 15>(p));
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        const uint4 va = Tl.v[2 * pr], vb = Tl.v[2 * pr + 1];
        const uint32_t wa[4] = {va.x, va.y, va.z, va.w};
        const uint32_t wb[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t even = __builtin_amdgcn_perm(wb[q], wa[q], 0x05040100u);  // dim 2q
          const uint32_t odd = __builtin_amdgcn_perm(wb[q], wa[q], 0x07060302u);   // dim 2q+1
#pragma unroll
          for (int h = 0; h < GM; ++h) {
            o[h][2 * q] = dot2(even, pp[h][pr], o[h][2 * q]);
            o[h][2 * q + 1] = dot2(odd, pp[h][pr], o[h][2 * q + 1]);
          }
        }
      }
    };

    // The workgroup's NW waves share the segment: wave wv takes tiles wv, wv + NW, ... . A ring
    // of kRing tile buffers keeps kRing - 1 tiles' loads in flight while one is consumed (this
    // prefetch depth, times the waves per SIMD, is what hides the memory latency).
    const int ntile = (seg + kTokens - 1) / kTokens;
    Tile ring[kRing];
#pragma unroll
    for (int i = 0; i < kRing - 1; ++i) load_tile(ring[i], wv + NW * i);
    for (int tile = wv; tile < ntile; tile += NW * kRing) {
#pragma unroll
      for (int u = 0; u < kRing; ++u) {
        const int cur = tile + NW * u;
        if (cur >= ntile) break;
        load_tile(ring[(u + kRing - 1) % kRing], cur + NW * (kRing - 1));
        process(ring[u], cur);
      }
    }

    // Per-head totals of this wave: l summed over the four lanes of head c%4, then every lane
    // takes the (m, l) of all four heads of its row from its quad. Into LDS for the merge.
    l += dpp<kRowRor4>(l);
    l += dpp<kRowRor8>(l);
    WaveAcc &mine = s_acc[wv];
#pragma unroll
    for (int h = 0; h < GM; ++h) {
      *reinterpret_cast<float4 *>(&mine.o[r][h][c * 8]) = make_float4(o[h][0], o[h][1], o[h][2], o[h][3]);
      *reinterpret_cast<float4 *>(&mine.o[r][h][c * 8 + 4]) = make_float4(o[h][4], o[h][5], o[h][6], o[h][7]);
    }
    if (c < GM) {  // lane c of the row holds head c's (m, l)
      mine.m[r][c] = m;
      mine.l[r][c] = l;
    }
    lds_barrier();  // not __syncthreads(): its global fence would wait for the prefetch past
                    // the segment; the waves share nothing through global memory

    // Merge the waves: wave wv now owns KV-head row wv % 4 and, with eight waves, half of its
    // dims; lane (h, c) = (lane / 16, lane % 16) owns head h and kMergeDims dims from d0.
    const int mr = wv % KG;
    const int mh = lane >> 4;
    const int d0 = (wv / KG) * (D / kMergeSplit) + c * kMergeDims;
    float M = -INFINITY;
#pragma unroll
    for (int u = 0; u < NW; ++u) M = fmaxf(M, s_acc[u].m[mr][mh]);
    float L = 0.f, acc[kMergeDims];
#pragma unroll
    for (int e = 0; e < kMergeDims; ++e) acc[e] = 0.f;
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const float wgt = exp2_or_zero(s_acc[u].m[mr][mh] - M);
      L += s_acc[u].l[mr][mh] * wgt;
#pragma unroll
      for (int e4 = 0; e4 < kMergeDims; e4 += 4) {
        const float4 a = *reinterpret_cast<const float4 *>(&s_acc[u].o[mr][mh][d0 + e4]);
        acc[e4 + 0] = fmaf(a.x, wgt, acc[e4 + 0]);
        acc[e4 + 1] = fmaf(a.y, wgt, acc[e4 + 1]);
        acc[e4 + 2] = fmaf(a.z, wgt, acc[e4 + 2]);
        acc[e4 + 3] = fmaf(a.w, wgt, acc[e4 + 3]);
      }
    }

    // This row's output heads (a row past H_kv writes nothing).
    const int m_kvh = kg * KG + mr;
    const bool m_live = m_kvh < P.H_kv && mh < min(GM, P.G - hc * GM);
    uint16_t *out_at = P.out + (int64_t(b) * P.H + int64_t(m_kvh) * P.G + hc * GM + mh) * D + d0;
    auto write_out = [&](const float (&v)[kMergeDims], float denom) {
      const float inv = 1.f / denom;
      uint32_t w[kMergeDims / 2];
#pragma unroll
      for (int e = 0; e < kMergeDims / 2; ++e) w[e] = pack_bf16(v[2 * e] * inv, v[2 * e + 1] * inv);
      if constexpr (kMergeDims == 8)
        *reinterpret_cast<uint4 *>(out_at) = make_uint4(w[0], w[1], w[2], w[3]);
      else
        *reinterpret_cast<uint2 *>(out_at) = make_uint2(w[0], w[1]);
    };

    // The ring's registers stay allocated to it up to here, after the four-wave merge: the
    // loads of the tile prefetched past the segment may still be in flight, and code that
    // reused those registers earlier would have to wait for them first.
#pragma unroll
    for (int i = 0; i < kRing; ++i) keep_tile(ring[i], acc[0]);

    const int ug = b * P.n_units + unit;
    const int64_t unit_start = Pb + int64_t(unit) * span + kSegCost;  // slot of its first key
    const int g_first = group_of(unit_start, T, NG);
    const int g_last = group_of(unit_start + nk - 1, T, NG);
    // The workgroup holding the unit's first key tells the merge pass where the unit's
    // partials are, so that it need not rebuild the work split from cache_seqlens.
    if (g == g_first && threadIdx.x == 0) P.desc[ug] = make_int2(g_first, g_last - g_first + 1);
    if (g_first == g_last && P.n_pre == 0) {
      if (m_live) write_out(acc, L);  // the segment is the whole unit
    } else {
      // This workgroup's partial for the unit, segment j = g - g_first: bucket slot j of the
      // unit, or overflow slot g + ug (distinct for every segment: the next unit's first
      // workgroup is at least this unit's last). The merge kernel, launched next on the same
      // stream, combines a unit's partials.
      const int j = g - g_first;
      char *slot = j < kBucket ? P.part + (int64_t(ug) * kBucket + j) * kSlot
                               : P.over + int64_t(g + ug) * kSlot;
      uint32_t w[kMergeDims / 2];
#pragma unroll
      for (int e = 0; e < kMergeDims / 2; ++e) w[e] = pack_bf16(acc[2 * e], acc[2 * e + 1]);
      char *po = slot + ((mr * GM + mh) * D + d0) * 2;
      if constexpr (kMergeDims == 8)
        *reinterpret_cast<uint4 *>(po) = make_uint4(w[0], w[1], w[2], w[3]);
      else
        *reinterpret_cast<uint2 *>(po) = make_uint2(w[0], w[1]);
      if (c == 0 && wv < KG)
        *reinterpret_cast<float2 *>(slot + kSlotO + 8 * (mr * GM + mh)) = make_float2(M, L);
    }
    lds_barrier();  // s_acc is reused by the next segment

    // Next segment: the next unit of this row, or the next row that has keys.
    x += seg;
    if (x == Pb + int64_t(span) * P.n_units) {
      Pb = x;
      int lo2;
      do {
        ++b;
      } while (b < P.B && row_keys_at(P, row_pos(b), lo2) == 0);
    }
  }
}

template <bool NT>
__global__ __launch_bounds__(64 * NW) void decode_fused_kernel(
    const int32_t *a_seqlens, const uint16_t *a_q, uint16_t *a_k_cache, uint16_t *a_v_cache,
    int a_B, int a_n_groups, int a_window, int a_lo_floor, int a_T_max, int a_n_units,
    FusedParams P) {
  decode_fused_body<NT, false>(a_seqlens, a_q, a_k_cache, a_v_cache, a_B, a_n_groups, a_window,
                               a_lo_floor, a_T_max, a_n_units, P, nullptr);
}

// The same pass with the shared prefix's jobs beside it: at most 256 registers per lane, so that
// a job's workgroup and a streaming one share a compute unit.
template <bool NT>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void
decode_fused_prefix_kernel(const int32_t *a_seqlens, const uint16_t *a_q, uint16_t *a_k_cache,
                           uint16_t *a_v_cache, int a_B, int a_n_groups, int a_window,
                           int a_lo_floor, int a_T_max, int a_n_units, FusedParams P,
                           px::Params X) {
  decode_fused_body<NT, true>(a_seqlens, a_q, a_k_cache, a_v_cache, a_B, a_n_groups, a_window,
                              a_lo_floor, a_T_max, a_n_units, P, &X);
}

// Merge pass with one wave per (unit, query head): lane l combines dims 2l, 2l+1 of that head
// over the unit's segments. The loads of the unit's first SPEC bucket slots are issued with that
// of its descriptor, before the segment count is known (one memory round trip for units of up to
// SPEC segments; slots past the count hold other calls' data and are ignored); later segments
// follow BATCH at a time. The pass does not read cache_seqlens (the descriptors carry all it
// needs), so it can also advance the positions: the wave of each row's first unit and head adds
// `advance` to the row's entry.
// NP > 0: also fold in the unit's n_pre <= NP partials of the shared prefix (loaded with the
// rest, in the same round trip); a unit's single segment is then a partial too.
// As for the streaming pass, the leading arguments are the fields of P the pass needs first,
// passed separately so that they arrive preloaded in SGPRs.
template <int SPEC, int NP>
__global__ __launch_bounds__(64) void decode_merge_kernel(
    const char *__restrict__ a_part, const int2 *__restrict__ a_desc, uint16_t *a_out,
    int32_t *a_adv, int a_n_units, int a_n_hc, int a_H_kv, int a_G, int a_H, int a_advance,
    FusedParams P) {
  P.part = const_cast<char *>(a_part);
  P.desc = const_cast<int2 *>(a_desc);
  P.out = a_out;
  P.adv_seqlens = a_adv;
  P.n_units = a_n_units;
  P.n_hc = a_n_hc;
  P.H_kv = a_H_kv;
  P.G = a_G;
  P.H = a_H;
  P.advance = a_advance;
  constexpr int BATCH = 8;
  const int lane = threadIdx.x;
  const int ug = blockIdx.x / (KG * GM);
  const int hr = blockIdx.x - ug * (KG * GM);  // KV row * GM + head within the unit
  const int b = ug / P.n_units;
  const int unit = ug - b * P.n_units;
  const int kg = unit / P.n_hc;
  const int hc = unit - kg * P.n_hc;
  const int kvh = kg * KG + hr / GM;
  const int hh = hr % GM;
  // An atomic add whose result is not used: the wave does not wait for a read of the position
  // before its own loads (one wave and lane per row adds, so it is a plain increment).
  if (P.advance != 0 && unit == 0 && hr == 0 && lane == 0) atomicAdd(P.adv_seqlens + b, P.advance);
  if (kvh >= P.H_kv || hh >= min(GM, P.G - hc * GM)) return;
  const char *bucket = P.part + int64_t(ug) * kBucket * kSlot;
  auto seg_at = [&](int j, int g_first) -> const char * {
    return j < kBucket ? bucket + int64_t(j) * kSlot : P.over + int64_t(g_first + j + ug) * kSlot;
  };
  // (m, l) and this lane's two dims of o (bf16) of head hr in a slot.
  auto slot_ml = [&](const char *ps) {
    return *reinterpret_cast<const float2 *>(ps + kSlotO + 8 * hr);
  };
  auto slot_v = [&](const char *ps) {
    const uint32_t o2 = *reinterpret_cast<const uint32_t *>(ps + (hr * D + 2 * lane) * 2);
    return make_float2(__uint_as_float(o2 << 16), __uint_as_float(o2 & 0xffff0000u));
  };
  // The unit's (first workgroup, segments), published by the streaming pass: no segments for a
  // row outside the cache (its NaN output is written), one for a unit written directly.
  const int2 d = P.desc[ug];
  float2 ml[SPEC], v[SPEC];
#pragma unroll
  for (int k = 0; k < SPEC; ++k) {
    const char *ps = bucket + int64_t(k) * kSlot;
    ml[k] = slot_ml(ps);
    v[k] = slot_v(ps);
  }
  constexpr bool PRE = NP > 0;
  float2 pml[PRE ? NP : 1], pv[PRE ? NP : 1];
  if constexpr (PRE) {
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const char *ps = P.pre + (int64_t(ug) * P.n_pre + min(k, P.n_pre - 1)) * kSlot;
      pml[k] = slot_ml(ps);
      pv[k] = slot_v(ps);
    }
  }
  // The loads above stay ahead of the branch below: the compiler would otherwise sink them past
  // it and issue them only once the descriptor is back (two memory round trips, not one).
#pragma unroll
  for (int k = 0; k < SPEC; ++k) asm volatile("" ::"v"(ml[k]), "v"(v[k]));
  if constexpr (PRE) {
#pragma unroll
    for (int k = 0; k < NP; ++k) asm volatile("" ::"v"(pml[k]), "v"(pv[k]));
  }
  const int g_first = d.x, nseg = d.y;
  // No keys (a row outside the cache: NaN written), or a unit written directly.
  if (nseg == 0 || (!PRE && nseg == 1)) return;
  // The slots loaded up front in two passes: their maximum, then each weighted against it (the
  // weights independent of one another, not a chain of rescales); later segments online.
  float M = -INFINITY, L = 0.f, t0 = 0.f, t1 = 0.f;
#pragma unroll
  for (int k = 0; k < SPEC; ++k)
    if (k < nseg) M = fmaxf(M, ml[k].x);
  if constexpr (PRE) {
#pragma unroll
    for (int k = 0; k < NP; ++k)
      if (k < P.n_pre) M = fmaxf(M, pml[k].x);
  }
  auto weigh = [&](float2 mlk, float2 vk, bool valid) {
    const float w = valid ? exp2_or_zero(mlk.x - M) : 0.f;
    L = fmaf(valid ? mlk.y : 0.f, w, L);
    t0 = fmaf(valid ? vk.x : 0.f, w, t0);
    t1 = fmaf(valid ? vk.y : 0.f, w, t1);
  };
#pragma unroll
  for (int k = 0; k < SPEC; ++k) weigh(ml[k], v[k], k < nseg);
  if constexpr (PRE) {
#pragma unroll
    for (int k = 0; k < NP; ++k) weigh(pml[k], pv[k], k < P.n_pre);
  }
  auto add = [&](float2 mlk, float2 vk, bool valid) {
    const float mk = valid ? mlk.x : -INFINITY;
    const float m_new = fmaxf(M, mk);
    const float fa = exp2_or_zero(M - m_new), fb = exp2_or_zero(mk - m_new);
    L = L * fa + (valid ? mlk.y : 0.f) * fb;
    t0 = t0 * fa + (valid ? vk.x : 0.f) * fb;
    t1 = t1 * fa + (valid ? vk.y : 0.f) * fb;
    M = m_new;
  };
  for (int s0 = SPEC; s0 < nseg; s0 += BATCH) {
    float2 mb[BATCH], vb[BATCH];
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const char *ps = seg_at(min(s0 + k, nseg - 1), g_first);
      mb[k] = slot_ml(ps);
      vb[k] = slot_v(ps);
    }
#pragma unroll
    for (int k = 0; k < BATCH; ++k) add(mb[k], vb[k], s0 + k < nseg);
  }
  const float inv = 1.f / L;
  *reinterpret_cast<uint32_t *>(P.out + (int64_t(b) * P.H + int64_t(kvh) * P.G + hc * GM + hh) * D +
                                2 * lane) = pack_bf16(t0 * inv, t1 * inv);
}

// Number of compute units of the current device, queried once per device. Threads that race on
// the first query each store the same value; the atomics make that well-defined.
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace

int64_t decode_fused_units(int64_t n_head, int64_t n_kv_head) {
  const int64_t G = n_head / n_kv_head;
  return ((n_kv_head + KG - 1) / KG) * ((G + GM - 1) / GM);
}

size_t decode_fused_partial_bytes(int64_t batch, int64_t n_head, int64_t n_kv_head,
                                  int64_t t_max, int64_t window) {
  (void)t_max;
  (void)window;
  const int64_t units = batch * decode_fused_units(n_head, n_kv_head);
  return size_t((units * kBucket + kMaxGroups + units) * kSlot + units * int64_t(sizeof(int2)));
}

size_t decode_prefix_bytes(int64_t batch, int64_t n_head, int64_t n_kv_head, int64_t head_dim,
                           int64_t t_max, int64_t window) {
  // Worth it for many queries per KV head (rows x query heads fill most of the matrix-core
  // kernel's 256 pairs) and without a window (its keys would then differ per row); possible only
  // for geometries the matrix-core kernel takes.
  if (head_dim != D || window >= 0 || n_kv_head <= 0 || batch * (n_head / n_kv_head) < 64 ||
      !prefill_mfma_geometry_ok(n_head, n_kv_head, t_max))
    return 0;
  const int64_t units = batch * decode_fused_units(n_head, n_kv_head);
  return size_t(units * kPrefixMaxSplits * kSlot);
}

bool decode_fused_supported(const AttnArgs &a) {
  // The merge grid has one wave per (unit, query head of a unit): it must fit a 32-bit grid.
  return a.dtype == MCAMD_BF16 && a.head_dim == D &&
         a.batch * decode_fused_units(a.n_head, a.n_kv_head) * KG * GM < (int64_t(1) << 31);
}

int launch_decode_fused(const AttnArgs &a) {
  FusedParams P;
  P.q = static_cast<const uint16_t *>(a.q);
  P.k_new = static_cast<const uint16_t *>(a.k_new);
  P.v_new = static_cast<const uint16_t *>(a.v_new);
  P.k_cache = static_cast<uint16_t *>(const_cast<void *>(a.k_cache));
  P.v_cache = static_cast<uint16_t *>(const_cast<void *>(a.v_cache));
  P.seqlens = a.seqlens;
  P.adv_seqlens = a.advance_seqlens;
  P.advance = a.advance_seqlens ? a.advance : 0;
  P.shared = int(std::min<int64_t>(std::max<int64_t>(a.shared_prefix, 0), a.t_max));
  P.out = static_cast<uint16_t *>(a.out);
  P.B = int(a.batch);
  P.H = int(a.n_head);
  P.H_kv = int(a.n_kv_head);
  P.G = int(a.n_head / a.n_kv_head);
  P.n_hc = (P.G + GM - 1) / GM;
  P.n_kg = (P.H_kv + KG - 1) / KG;
  P.n_units = P.n_kg * P.n_hc;
  P.T_max = int(a.t_max);
  P.window = int(a.window < 0 ? -1 : a.window);
  P.cache_b = a.cache_batch_stride;
  // Row slot counts are at most (T_max + kSegCost) * n_units each.
  P.scan32 = a.batch <= 64 &&
             a.batch * P.n_units * (a.t_max + int64_t(kSegCost)) < (int64_t(1) << 31);
  P.scale_log2 = float(kLog2e / std::sqrt(double(D)));
  // Workgroups: one per CU, but no more than one per kMinKeysPerGroup slots of the largest total.
  const int64_t span = a.window >= 0 ? std::min<int64_t>(a.t_max, a.window + 1) : a.t_max;
  const int64_t t_upper = a.batch * P.n_units * span;
  int64_t groups = std::min<int64_t>(int64_t(device_cus()) * kGroupsPerCU, kMaxGroups);
  groups = std::max<int64_t>(1, std::min<int64_t>(groups, (t_upper + kMinKeysPerGroup - 1) / kMinKeysPerGroup));
  P.n_groups = int(groups);
  char *ws = static_cast<char *>(a.workspace);
  const int64_t units = int64_t(P.B) * P.n_units;
  P.part = ws;
  P.over = P.part + units * kBucket * kSlot;
  P.desc = reinterpret_cast<int2 *>(P.over + (kMaxGroups + units) * kSlot);
  // A long shared prompt prefix of a wide batch goes to the matrix cores (every row's queries
  // against row 0's prefix keys at once, in key ranges) when the workspace has room for those
  // partials; this pass then covers each row's own keys only, and the merge folds both.
  P.lo_floor = 0;
  P.pre = nullptr;
  P.n_pre = 0;
  px::Params X{};  // the prefix jobs (P.n_pre > 0)
  const size_t base_ws =
      decode_workspace_bytes(a.batch, a.n_head, a.n_kv_head, a.head_dim, a.t_max, a.window);
  const size_t pre_ws =
      decode_prefix_bytes(a.batch, a.n_head, a.n_kv_head, a.head_dim, a.t_max, a.window);
  if (pre_ws > 0 && a.shared_prefix >= kPrefixMinKeys && a.workspace_bytes >= base_ws + pre_ws) {
    P.n_pre = px::splits(a.batch, a.n_head, a.n_kv_head, a.shared_prefix, device_cus(),
                         kPrefixMaxSplits);
    P.lo_floor = int(a.shared_prefix);
    char *pre = ws + base_ws;
    P.pre = pre;
    X.q = static_cast<const uint16_t *>(a.q);
    X.k_cache = static_cast<const uint16_t *>(a.k_cache);
    X.v_cache = static_cast<const uint16_t *>(a.v_cache);
    X.part = pre;
    X.H = P.H;
    X.H_kv = P.H_kv;
    X.G = P.G;
    X.n_pairs = P.B * P.G;
    X.n_pb = (X.n_pairs + px::kPairsPerJob - 1) / px::kPairsPerJob;
    X.n_split = P.n_pre;
    X.key_len = int((a.shared_prefix + P.n_pre - 1) / P.n_pre);
    X.prefix = int(a.shared_prefix);
    X.n_units = P.n_units;
    X.n_hc = P.n_hc;
    X.T_max = P.T_max;
    X.scale_log2 = P.scale_log2;
    X.jobs = X.n_pb * P.H_kv * P.n_pre;
    // Every key range holds keys: (n_pre - 1) * ceil(prefix / n_pre) < prefix, since at most
    // sixteen ranges of at least 128 keys are made.
    if (int64_t(P.n_pre - 1) * X.key_len >= a.shared_prefix)
      return fail(MCAMD_EINVAL, "decode: empty shared-prefix key range");
  }
  // K/V bytes the call can read (every row at its longest span). A call that fits in a quarter
  // of the 256 MB memory-side cache loads them with the default policy, so a KV-sharing layer
  // that reads the same slot next finds them there (measured on the 24-layer mixed-window stack:
  // 0.413 -> 0.393 ms per step; the same for its global calls too: 0.412, no gain). Larger calls
  // stream non-temporal: allocating lines that no later read finds costs bandwidth (the decode
  // microbench's call with the default policy, alternating two caches: 57.3 against 49.8 us).
  const int64_t kv_bytes = int64_t(a.batch) * span * a.n_kv_head * D * 2 * 2;
  auto stream_pass = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(unsigned(groups)), dim3(64 * NW), 0, a.stream, P.seqlens, P.q,
                       P.k_cache, P.v_cache, P.B, P.n_groups, P.window, P.lo_floor, P.T_max,
                       P.n_units, P);
  };
  // With a prefix on the matrix cores, its jobs are the grid's last workgroups.
  auto prefix_pass = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(unsigned(groups + X.jobs)), dim3(64 * NW), 0, a.stream,
                       P.seqlens, P.q, P.k_cache, P.v_cache, P.B, P.n_groups, P.window,
                       P.lo_floor, P.T_max, P.n_units, P, X);
  };
  const bool nt = kv_bytes > kTemporalLimit;
  if (P.n_pre > 0)
    nt ? prefix_pass(decode_fused_prefix_kernel<true>) : prefix_pass(decode_fused_prefix_kernel<false>);
  else
    nt ? stream_pass(decode_fused_kernel<true>) : stream_pass(decode_fused_kernel<false>);
  int st = launch_status("decode_fused");
  if (st != MCAMD_OK) return st;
  const dim3 merge_grid(unsigned(a.batch * P.n_units * KG * GM));
  // Speculative slot loads sized to the segments a unit is expected to have (about one per
  // workgroup its keys span, plus the ends): the units of a wide batch span few workgroups, and
  // loading sixteen slots for them would read mostly unused partials (measured on the 64-row,
  // 32-layer sampling decode: 6.71 -> 6.62 ms per step with 4 slots; 16 kept where units span
  // many workgroups, as in the 32-row microbench and the mixed-window stack).
  const int64_t per_unit = groups / std::max<int64_t>(1, units) + 2;
  auto merge = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, merge_grid, dim3(64), 0, a.stream, P.part, P.desc, P.out,
                       P.adv_seqlens, P.n_units, P.n_hc, P.H_kv, P.G, P.H, P.advance, P);
  };
  constexpr int S16 = kSpec < 16 ? kSpec : 16, S8 = kSpec < 8 ? kSpec : 8,
                S4 = kSpec < 4 ? kSpec : 4;
  if (P.n_pre > 8)
    merge(decode_merge_kernel<S4, kPrefixMaxSplits>);
  else if (P.n_pre > 4)
    merge(decode_merge_kernel<S4, 8>);
  else if (P.n_pre > 0)
    merge(decode_merge_kernel<S4, 4>);
  else if (kSpec >= 16 && per_unit > 8)
    merge(decode_merge_kernel<S16, 0>);
  else if (per_unit > 4)
    merge(decode_merge_kernel<S8, 0>);
  else
    merge(decode_merge_kernel<S4, 0>);
  return launch_status("decode_merge");
}

}  // namespace mcamd
