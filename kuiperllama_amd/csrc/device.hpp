// Device helpers shared by the op-level and fused decode kernels (gfx950,
// wave64).  Vector types are clang ext_vector types so that 16-byte loads can
// carry the nontemporal hint.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kl {

typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int i4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kBlock = 256;  // four wave64s per workgroup
constexpr int kWavesPerBlock = kBlock / kWave;

// Streaming (read-once) weight loads: the nontemporal hint keeps them from
// evicting the small, reused activation vectors from the caches.
__device__ __forceinline__ f4 load_stream(const f4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ i4 load_stream(const i4* p) { return __builtin_nontemporal_load(p); }

__device__ __forceinline__ float hsum(f4 v) { return (v.x + v.y) + (v.z + v.w); }

// Butterfly sum over all 64 lanes; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Sum over groups of `width` consecutive lanes (width a power of two <= 64).
__device__ __forceinline__ float group_sum(float v, int width) {
  for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Block-wide sum for a 256-thread block; `red` is LDS scratch of >= 4 floats.
// Every thread receives the total.  Contains barriers: call uniformly.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kWavesPerBlock; ++w) t += red[w];
  return t;
}

// (value, index) argmax with the reference's tie rule: the lower index wins
// among equal values (std::max_element keeps the first maximum).
__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(v, off, kWave);
    const int oi = __shfl_xor(i, off, kWave);
    argmax_merge(v, i, ov, oi);
  }
}

// Cross-workgroup hand-off without cache maintenance.  The L2 of an MI355X
// XCD is not coherent with the other XCDs' L2s, and a device-scope fence
// (__threadfence) writes back and invalidates the whole L2.  Instead, the few
// words one workgroup passes to another go through agent-coherent (sc1)
// stores and loads, the producer waits for its stores to complete
// (wait_mem) before a device-scope atomic announces them, and the consumer,
// having observed the atomic, reads them with coherent loads.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int load_coherent(const int* p) {
  return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until every memory operation this wave issued has completed.
__device__ __forceinline__ void wait_mem() { __builtin_amdgcn_s_waitcnt(0); }
// Device-scope arrival counter; returns the previous value.
__device__ __forceinline__ unsigned int arrive(unsigned int* counter) {
  return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// RoPE rotation of one pair, written without contraction so that the result
// is the same float expression the reference CPU path evaluates
// (kernels/cpu/rope_kernel.cpp:37-38 / :115-118): v0*c - v1*s, v0*s + v1*c.
__device__ __forceinline__ void rope_pair(float& v0, float& v1, float fcr, float fci) {
#pragma clang fp contract(off)
  const float a = v0 * fcr - v1 * fci;
  const float b = v0 * fci + v1 * fcr;
  v0 = a;
  v1 = b;
}

// Signed bytes of a dword as floats.
__device__ __forceinline__ void unpack_i8x4(int w, float* o) {
  o[0] = static_cast<float>((w << 24) >> 24);
  o[1] = static_cast<float>((w << 16) >> 24);
  o[2] = static_cast<float>((w << 8) >> 24);
  o[3] = static_cast<float>(w >> 24);
}

}  // namespace kl
