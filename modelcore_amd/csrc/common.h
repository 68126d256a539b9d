// Shared device and host helpers for the modelcore_amd HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/modelcore_amd.h"

namespace mcamd {

// ---------------------------------------------------------------------------------------------
// Host-side error reporting: one thread-local message, read through mcamd_last_error().
// ---------------------------------------------------------------------------------------------
void set_error(const std::string &msg);
void clear_error();

inline int fail(int code, const std::string &msg) {
  set_error(msg);
  return code;
}

// Turns the status of the last launch into an ABI status.
inline int launch_status(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(MCAMD_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  clear_error();
  return MCAMD_OK;
}

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void *p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

// ---------------------------------------------------------------------------------------------
// Element types. Storage is what sits in HBM; arithmetic is always fp32.
// ---------------------------------------------------------------------------------------------
struct bf16 {
  uint16_t bits;
};

// bf16 <-> fp32. Widening is exact (bf16 is the top half of an fp32). Narrowing rounds to
// nearest, ties to even, and keeps NaN a (quiet) NaN.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b16) {
  return __uint_as_float(b16 << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// A 16-byte load marked non-temporal (the `nt` cache policy): for data read once per pass, such
// as K/V streamed by decode attention. The lines are not kept in L2 or the memory-side cache, so
// they neither evict data that is reused nor make a repeated benchmark look faster than the same
// pass over a cold cache (measured: without it, re-reading one 285 MB cache ran 12% faster than
// rotating over distinct ones; with it, both run alike).
typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream(const void *p) {
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load(static_cast<const u32x4_nt *>(p)));
}

// A workgroup barrier that orders LDS accesses only. __syncthreads() also fences global memory,
// so the waves first wait for every global load and store they have in flight; where a
// workgroup's waves share nothing through global memory, that wait is pure latency.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// A 16-byte vector of elements: 8 x bf16 or 4 x fp32. All kernels move data in these units.
template <class E> struct Vec;

template <> struct Vec<bf16> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void load(const bf16 *p, float (&x)[8]) {
    uint4 u = *reinterpret_cast<const uint4 *>(p);
    x[0] = __uint_as_float(u.x << 16);
    x[1] = __uint_as_float(u.x & 0xffff0000u);
    x[2] = __uint_as_float(u.y << 16);
    x[3] = __uint_as_float(u.y & 0xffff0000u);
    x[4] = __uint_as_float(u.z << 16);
    x[5] = __uint_as_float(u.z & 0xffff0000u);
    x[6] = __uint_as_float(u.w << 16);
    x[7] = __uint_as_float(u.w & 0xffff0000u);
  }
  __device__ __forceinline__ static void unpack(const uint4 &u, float (&x)[8]) {
    x[0] = __uint_as_float(u.x << 16);
    x[1] = __uint_as_float(u.x & 0xffff0000u);
    x[2] = __uint_as_float(u.y << 16);
    x[3] = __uint_as_float(u.y & 0xffff0000u);
    x[4] = __uint_as_float(u.z << 16);
    x[5] = __uint_as_float(u.z & 0xffff0000u);
    x[6] = __uint_as_float(u.w << 16);
    x[7] = __uint_as_float(u.w & 0xffff0000u);
  }
  __device__ __forceinline__ static void store(bf16 *p, const float (&x)[8]) {
    uint4 u;
    u.x = f32_to_bf16_bits(x[0]) | (uint32_t(f32_to_bf16_bits(x[1])) << 16);
    u.y = f32_to_bf16_bits(x[2]) | (uint32_t(f32_to_bf16_bits(x[3])) << 16);
    u.z = f32_to_bf16_bits(x[4]) | (uint32_t(f32_to_bf16_bits(x[5])) << 16);
    u.w = f32_to_bf16_bits(x[6]) | (uint32_t(f32_to_bf16_bits(x[7])) << 16);
    *reinterpret_cast<uint4 *>(p) = u;
  }
};

template <> struct Vec<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void load(const float *p, float (&x)[4]) {
    float4 u = *reinterpret_cast<const float4 *>(p);
    x[0] = u.x;
    x[1] = u.y;
    x[2] = u.z;
    x[3] = u.w;
  }
  __device__ __forceinline__ static void unpack(const uint4 &u, float (&x)[4]) {
    x[0] = __uint_as_float(u.x);
    x[1] = __uint_as_float(u.y);
    x[2] = __uint_as_float(u.z);
    x[3] = __uint_as_float(u.w);
  }
  __device__ __forceinline__ static void store(float *p, const float (&x)[4]) {
    *reinterpret_cast<float4 *>(p) = make_float4(x[0], x[1], x[2], x[3]);
  }
};

template <class E> __device__ __forceinline__ float to_f32(E x);
template <> __device__ __forceinline__ float to_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ float to_f32<bf16>(bf16 x) { return bf16_bits_to_f32(x.bits); }

template <class E> __device__ __forceinline__ E from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return bf16{f32_to_bf16_bits(x)}; }

// ---------------------------------------------------------------------------------------------
// Wave64 reductions.
// ---------------------------------------------------------------------------------------------
template <int WIDTH>
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}
template <int WIDTH>
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

// The power of two (16 to 256) whose kernel instantiation serves head_dim d, or 0 past 256.
inline int head_dim_bucket(int64_t d) {
  if (d > 512) return 0;
  int p = 16;
  while (p < d) p *= 2;
  return p;
}

// Key range of the query at position p under a left window (w < 0 = unlimited): [lo, p].
__device__ __forceinline__ int key_lo(int p, int window) {
  return window >= 0 ? max(0, p - window) : 0;
}

}  // namespace mcamd
