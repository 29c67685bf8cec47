// Op-level C ABI: runtime (memory, streams, events) and one launcher per
// reference kernel typedef (kuiper/source/op/kernels/kernels_interface.h:6-47).
// Every launcher validates its arguments on the host, so a kernel is never
// launched with a shape it does not handle.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "attn.hpp"
#include "device.hpp"
#include "gemm.hpp"
#include "gemv.hpp"
#include "prefill.hpp"
#include "kuiper_hip.h"

using namespace kl;

namespace {

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }
inline int rc(hipError_t e) { return e == hipSuccess ? KL_OK : static_cast<int>(e); }
inline int launch_rc() { return rc(hipGetLastError()); }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------
// GEMV (MatmulKernel / MatmulKernelQuant).
// ---------------------------------------------------------------------------
// Vector path: run_tiles() with x read straight from global memory (it is
// small and cache resident), one wave per (row, 8 KiB slice).
template <bool Q8, int U>
__global__ __launch_bounds__(512) void k_gemv(const float* __restrict__ x, WView w, ColGeom g,
                                             float* __restrict__ y, int rows, float scale) {
  __shared__ float red[32];
  auto rowfn = [&](int u, int, WView& m, size_t& row) {
    m = w;
    row = u;
  };
  auto stage = [] {};
  auto epi = [&](int u, const float (&v)[1]) {
    if ((threadIdx.x & 63) == 0) y[u] = v[0] * scale;
  };
  run_tiles<Q8, 1, U>(g, rows, x, red, rowfn, stage, epi);
}

int launch_gemv(const float* x, WView w, float* y, int rows, int cols, bool q8, int group_size,
                float scale, hipStream_t s) {
  ColGeom g = make_geom(cols, q8, 4, group_size);
  int U = 4;
  if (g.ks > kMaxKs) {
    g = make_geom(cols, q8, 8, group_size);
    U = 8;
  }
  if (g.ks > kMaxKs) return KL_EUNSUPP;
  const int G = row_groups_for(g.ks);
  const int grid = std::max(1, std::min((rows + G - 1) / G, 8192));
  const dim3 block(kWave * g.ks * G);
  if (q8) {
    if (U == 8) hipLaunchKernelGGL((k_gemv<true, 8>), dim3(grid), block, 0, s, x, w, g, y, rows, scale);
    else hipLaunchKernelGGL((k_gemv<true, 4>), dim3(grid), block, 0, s, x, w, g, y, rows, scale);
  } else {
    if (U == 8) hipLaunchKernelGGL((k_gemv<false, 8>), dim3(grid), block, 0, s, x, w, g, y, rows, scale);
    else hipLaunchKernelGGL((k_gemv<false, 4>), dim3(grid), block, 0, s, x, w, g, y, rows, scale);
  }
  return launch_rc();
}

// Any shape / alignment: one wave per row, scalar loads.
__global__ __launch_bounds__(256) void k_gemv_f32_scalar(const float* __restrict__ x,
                                                        const float* __restrict__ W,
                                                        float* __restrict__ y, int rows, int cols,
                                                        float scale) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int r = blockIdx.x * kWavesPerBlock + wave; r < rows; r += gridDim.x * kWavesPerBlock) {
    const float* wr = W + static_cast<size_t>(r) * cols;
    float acc = 0.f;
    for (int c = lane; c < cols; c += kWave) acc += wr[c] * x[c];
    acc = wave_sum(acc);
    if (lane == 0) y[r] = acc * scale;
  }
}

// Any group size: per element (x * s) * q as the reference evaluates it.
__global__ __launch_bounds__(256) void k_gemv_q8_scalar(const float* __restrict__ x,
                                                       const int8_t* __restrict__ W,
                                                       const float* __restrict__ S,
                                                       float* __restrict__ y, int rows, int cols,
                                                       int gs) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int r = blockIdx.x * kWavesPerBlock + wave; r < rows; r += gridDim.x * kWavesPerBlock) {
    const size_t base = static_cast<size_t>(r) * cols;
    float acc = 0.f;
    for (int c = lane; c < cols; c += kWave) {
      const size_t idx = base + c;
      acc += (x[c] * S[idx / gs]) * static_cast<float>(W[idx]);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[r] = acc;
  }
}

__global__ void k_dequant_q8(const int8_t* __restrict__ q, const float* __restrict__ s, int64_t n,
                             int gs, float* __restrict__ out) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    out[i] = s[i / gs] * static_cast<float>(q[i]);
}

// ---------------------------------------------------------------------------
// RMSNorm.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_rmsnorm_1(const float* __restrict__ x,
                                                   const float* __restrict__ w, float* y, int n,
                                                   float eps) {
  __shared__ float red[16];
  __shared__ float s_r;
  float ss = 0.f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int k = 0; k < static_cast<int>(blockDim.x >> 6); ++k) t += red[k];
    s_r = 1.f / sqrtf(t / static_cast<float>(n) + eps);
  }
  __syncthreads();
  const float r = s_r;
  for (int i = threadIdx.x; i < n; i += blockDim.x) y[i] = w[i] * (r * x[i]);
}

__global__ __launch_bounds__(256) void k_rmsnorm_rows(const float* __restrict__ x,
                                                     const float* __restrict__ w, float* y,
                                                     int rows, int n, float eps) {
  __shared__ float red[kWavesPerBlock];
  const int row = blockIdx.x;
  const float* xr = x + static_cast<size_t>(row) * n;
  float* yr = y + static_cast<size_t>(row) * n;
  float ss = 0.f;
  for (int i = threadIdx.x; i < n; i += 256) ss += xr[i] * xr[i];
  ss = block_sum(ss, red);
  const float r = 1.f / sqrtf(ss / static_cast<float>(n) + eps);
  for (int i = threadIdx.x; i < n; i += 256) yr[i] = (r * xr[i]) * w[i];
}

// Rows of at most 1024 floats (n % 4 == 0, 16-byte aligned rows): one wave
// per row, float4 accesses, the sum of squares by lane exchanges only (no LDS,
// no barrier).  The per-head q/k norms of a prefill are 10^4+ such rows.
__global__ __launch_bounds__(256) void k_rmsnorm_rows_w(const float* __restrict__ x,
                                                       const float* __restrict__ w, float* y,
                                                       int rows, int n, float eps) {
  const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;  // whole waves
  const f4* xr = reinterpret_cast<const f4*>(x + static_cast<size_t>(row) * n);
  f4* yr = reinterpret_cast<f4*>(y + static_cast<size_t>(row) * n);
  const f4* w4 = reinterpret_cast<const f4*>(w);
  const int n4 = n / 4;
  f4 v[4];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = lane + j * kWave;
    v[j] = i < n4 ? xr[i] : f4{0.f, 0.f, 0.f, 0.f};
    ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
  }
  ss = wave_sum(ss);
  const float r = 1.f / sqrtf(ss / static_cast<float>(n) + eps);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = lane + j * kWave;
    if (i < n4) yr[i] = (r * v[j]) * w4[i];
  }
}

// Rows of up to 8192 floats (n % 4 == 0, 16-byte aligned): one block per
// row, each thread's float4s kept in registers between the sum of squares and
// the scaling, so the row is read once.
template <int R>
__global__ __launch_bounds__(256) void k_rmsnorm_rows_b(const float* __restrict__ x,
                                                       const float* __restrict__ w, float* y,
                                                       int rows, int n, float eps) {
  __shared__ float red[kWavesPerBlock];
  const int row = blockIdx.x;
  const f4* xr = reinterpret_cast<const f4*>(x + static_cast<size_t>(row) * n);
  f4* yr = reinterpret_cast<f4*>(y + static_cast<size_t>(row) * n);
  const f4* w4 = reinterpret_cast<const f4*>(w);
  const int n4 = n / 4;
  f4 v[R];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int i = threadIdx.x + j * 256;
    v[j] = i < n4 ? xr[i] : f4{0.f, 0.f, 0.f, 0.f};
    ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
  }
  ss = block_sum(ss, red);
  const float r = 1.f / sqrtf(ss / static_cast<float>(n) + eps);
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int i = threadIdx.x + j * 256;
    if (i < n4) yr[i] = (r * v[j]) * w4[i];
  }
}

// ---------------------------------------------------------------------------
// RoPE: one thread per rotated pair of q (and of k where the index < kv_dim).
// ---------------------------------------------------------------------------
// Pair p's two indices and its sin/cos table column.
__device__ __forceinline__ void rope_index(int style, int hd, int p, int& i0, int& i1, int& tab) {
  const int half = hd / 2;
  if (style == KL_ROPE_INTERLEAVED) {
    i0 = 2 * p;
    i1 = i0 + 1;
    tab = i0 % hd;
  } else {
    const int head = p / half, j = p - head * half;
    i0 = head * hd + j;
    i1 = i0 + half;
    tab = 2 * j;
  }
}

// Rotates pair p of q (and of k where the reference does) at position pos.
__device__ __forceinline__ void rope_one(int style, int kv_dim, int hd, float* q, float* k, int pos,
                                         int p, const float* __restrict__ sin_t,
                                         const float* __restrict__ cos_t) {
  int i0, i1, tab;
  rope_index(style, hd, p, i0, i1, tab);
  const float fci = sin_t[static_cast<size_t>(pos) * hd + tab];
  const float fcr = cos_t[static_cast<size_t>(pos) * hd + tab];
  float v0 = q[i0], v1 = q[i1];
  rope_pair(v0, v1, fcr, fci);
  q[i0] = v0;
  q[i1] = v1;
  // k is rotated where the pair's first q index (interleaved) or the head's
  // start (rotate-half) lies below kv_dim, as in the reference loops.
  const int gate = style == KL_ROPE_INTERLEAVED ? i0 : (i0 - (i0 % hd));
  if (gate < kv_dim) {
    float w0 = k[i0], w1 = k[i1];
    rope_pair(w0, w1, fcr, fci);
    k[i0] = w0;
    k[i1] = w1;
  }
}

__global__ void k_rope(int style, int dim, int kv_dim, int hd, float* q, float* k, int pos,
                       const float* __restrict__ sin_t, const float* __restrict__ cos_t) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p < dim / 2) rope_one(style, kv_dim, hd, q, k, pos, p, sin_t, cos_t);
}

// Rows r < n of q (stride ldq) and k (stride ldk) at positions pos0 + r.
__global__ void k_rope_rows(int style, int dim, int kv_dim, int hd, float* q, int ldq, float* k,
                            int ldk, int pos0, int n, const float* __restrict__ sin_t,
                            const float* __restrict__ cos_t) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  const int r = blockIdx.y;
  if (p < dim / 2 && r < n)
    rope_one(style, kv_dim, hd, q + static_cast<size_t>(r) * ldq, k + static_cast<size_t>(r) * ldk,
             pos0 + r, p, sin_t, cos_t);
}

// Qwen3's per-head q/k RMSNorm followed by RoPE on rows of a prefill, in one
// pass: HD / 4 lanes per (row, head) -- two heads per wave for head size 128,
// four for 64 -- q heads then k heads; lane l of a group holds the head's
// float4 l.  The norm is the one of k_rmsnorm_rows_w (sum of squares over the
// group's lanes in an xor butterfly, y = (r * x) * w); the rotation is
// rope_one's (rotate-half pairs (j, j + HD / 2) sit HD / 8 lanes apart and are
// exchanged across lanes; interleaved pairs lie within a float4), its cos/sin
// entries read as 16-byte vectors.  Every k head is rotated (they all lie
// below kv_dim).
template <int HD>
__global__ __launch_bounds__(256) void k_qk_norm_rope_rows(
    int style, int H, int KVH, float* q, int ldq, float* k, int ldk, const float* __restrict__ qn,
    const float* __restrict__ kn, float eps, int pos0, int n, const float* __restrict__ sin_t,
    const float* __restrict__ cos_t) {
  constexpr int C4 = HD / 4, PPW = kWave / C4;  // lanes per head, heads per wave
  static_assert(PPW * C4 == kWave && (HD / 8) * 2 == C4, "head size");
  const int heads = H + KVH;
  const long long total = static_cast<long long>(n) * heads;
  const int lane = threadIdx.x & 63, ll = lane % C4;
  const long long wid =
      (static_cast<long long>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6)) * PPW + lane / C4;
  const bool ok = wid < total;  // groups past the last (row, head) compute a clamped one, store nothing
  const long long pid = ok ? wid : total - 1;
  const int r = static_cast<int>(pid / heads), hh = static_cast<int>(pid - static_cast<long long>(r) * heads);
  const bool isq = hh < H;
  f4* x = reinterpret_cast<f4*>(isq ? q + static_cast<size_t>(r) * ldq + static_cast<size_t>(hh) * HD
                                    : k + static_cast<size_t>(r) * ldk + static_cast<size_t>(hh - H) * HD);
  const f4* w4 = reinterpret_cast<const f4*>(isq ? qn : kn);
  const f4 v = x[ll];
  float ss = v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  ss = group_sum(ss, C4);
  const float rn = 1.f / sqrtf(ss / static_cast<float>(HD) + eps);
  f4 y = (rn * v) * w4[ll];
  const size_t t0 = static_cast<size_t>(pos0 + r) * HD;
  if (style == KL_ROPE_HALF) {
    constexpr int OFF = HD / 8;  // lanes between the two halves of a pair
    const f4 pt = {__shfl_xor(y.x, OFF), __shfl_xor(y.y, OFF), __shfl_xor(y.z, OFF),
                   __shfl_xor(y.w, OFF)};
    const bool first = ll < OFF;
    const int jb = 4 * (first ? ll : ll - OFF);  // index of y.x within its half
    // entries t0 + 2 (jb + c), c = 0..3: the even ones of 8 consecutive floats
    const f4* ct = reinterpret_cast<const f4*>(cos_t + t0 + 2 * jb);
    const f4* st = reinterpret_cast<const f4*>(sin_t + t0 + 2 * jb);
    const f4 c0 = ct[0], c1 = ct[1], s0 = st[0], s1 = st[1];
    const float cs[4] = {c0.x, c0.z, c1.x, c1.z}, sn[4] = {s0.x, s0.z, s1.x, s1.z};
    float out[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float v0 = first ? y[c] : pt[c], v1 = first ? pt[c] : y[c];
      rope_pair(v0, v1, cs[c], sn[c]);
      out[c] = first ? v0 : v1;
    }
    y = f4{out[0], out[1], out[2], out[3]};
  } else {
    const int e = 4 * ll;  // element index of y.x within the head
    const f4 cs = *reinterpret_cast<const f4*>(cos_t + t0 + e);
    const f4 sn = *reinterpret_cast<const f4*>(sin_t + t0 + e);
    float a0 = y.x, a1 = y.y, b0 = y.z, b1 = y.w;
    rope_pair(a0, a1, cs.x, sn.x);
    rope_pair(b0, b1, cs.z, sn.z);
    y = f4{a0, a1, b0, b1};
  }
  if (ok) x[ll] = y;
}

// ---------------------------------------------------------------------------
// Elementwise.
// ---------------------------------------------------------------------------
__global__ void k_swiglu(const float* __restrict__ a, const float* __restrict__ b, float* out,
                         int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const float av = a[i];
    const float s = av * (1.0f / (1.0f + expf(-av)));
    out[i] = s * b[i];
  }
}

__global__ void k_add(const float* __restrict__ a, const float* __restrict__ b, float* out, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    out[i] = a[i] + b[i];
}

// ScaleKernel (cpu/scale_kernel.cpp:3-9): x = x * scale, one rounding.
__global__ void k_scale(float scale, float* x, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    x[i] = x[i] * scale;
}

// SoftmaxInplaceKernel (cpu/softmax_kernel.cpp:4-16) over one vector, one
// workgroup: the maximum (exact in any order), x = exp(x - max), their sum
// (in this workgroup's fixed tree order), x = x / sum.
__global__ __launch_bounds__(1024) void k_softmax_1(float* x, int n) {
  __shared__ float red[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  float m = -INFINITY;
  for (int i = tid; i < n; i += blockDim.x) m = fmaxf(m, x[i]);
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = red[0];
  for (int w = 1; w < nw; ++w) m = fmaxf(m, red[w]);
  __syncthreads();
  float s = 0.f;
  for (int i = tid; i < n; i += blockDim.x) {
    const float e = expf(x[i] - m);
    x[i] = e;
    s += e;
  }
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  s = red[0];
  for (int w = 1; w < nw; ++w) s += red[w];
  for (int i = tid; i < n; i += blockDim.x) x[i] = x[i] / s;
}

// ScaleSumKernel (cpu/scale_sum_kernel.cpp:5-22): out[d] += scale[i] * value[i
// * stride + d] for i = 0 .. pos in increasing i, the product and the sum each
// rounded (contraction into a fused multiply-add is off here), as the
// reference's vector expression does.
__global__ void k_scale_sum(const float* __restrict__ value, const float* __restrict__ scale,
                            float* out, int pos, int size, int stride) {
#pragma clang fp contract(off)
  for (int d = blockIdx.x * blockDim.x + threadIdx.x; d < size; d += gridDim.x * blockDim.x) {
    float acc = out[d];
    for (int i = 0; i <= pos; ++i) {
      const float p = scale[i] * value[static_cast<size_t>(i) * stride + d];
      acc = acc + p;
    }
    out[d] = acc;
  }
}

// One workgroup per token row.
__global__ __launch_bounds__(256) void k_embedding(const int32_t* __restrict__ tokens,
                                                  const float* __restrict__ table, int vocab,
                                                  int dim, float* __restrict__ out, int32_t* bad) {
  const int i = blockIdx.x;
  const int32_t t = tokens[i];
  if (t < 0 || t >= vocab) {
    if (threadIdx.x == 0 && bad) *bad = 1;
    return;
  }
  const float* src = table + static_cast<size_t>(t) * dim;
  float* dst = out + static_cast<size_t>(i) * dim;
  for (int c = threadIdx.x; c < dim; c += 256) dst[c] = src[c];
}

// ---------------------------------------------------------------------------
// Argmax: per-workgroup (value, index) partials, merged by the last workgroup
// to arrive (arrival counter reset by that workgroup).
// ---------------------------------------------------------------------------
constexpr int kArgmaxMaxBlocks = 1024;

// HBM read-bandwidth probe: one workgroup per CU streams its own contiguous
// chunk of `per` 16-byte elements, four loads in flight per thread, and keeps
// a running sum, stored once per thread so the loads are not dead code.
// (Measured on MI355X: 7.3 TB/s with one workgroup per CU against 6.0-6.4
// TB/s for a grid-stride loop over the whole buffer.)
__global__ __launch_bounds__(512) void k_read_probe(const kl::pf4* __restrict__ p, size_t per,
                                                     float* __restrict__ out) {
  const kl::pf4* q = p + static_cast<size_t>(blockIdx.x) * per;
  float acc = 0.f;
  size_t i = threadIdx.x;
  for (; i + 3 * 512 < per; i += 4 * 512) {
    const kl::pf4 a = __builtin_nontemporal_load(q + i);
    const kl::pf4 b = __builtin_nontemporal_load(q + i + 512);
    const kl::pf4 c = __builtin_nontemporal_load(q + i + 2 * 512);
    const kl::pf4 d = __builtin_nontemporal_load(q + i + 3 * 512);
    acc += ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)) +
           ((c.x + c.y) + (c.z + c.w)) + ((d.x + d.y) + (d.z + d.w));
  }
  for (; i < per; i += 512) {
    const kl::pf4 a = __builtin_nontemporal_load(q + i);
    acc += (a.x + a.y) + (a.z + a.w);
  }
  out[static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x] = acc;
}

__global__ __launch_bounds__(256) void k_argmax(const float* __restrict__ x, int n,
                                               int32_t* out_index, float* pv, int* pi,
                                               unsigned int* counter) {
  __shared__ float sv[kWavesPerBlock];
  __shared__ int si[kWavesPerBlock];
  __shared__ int s_last;
  float v = -INFINITY;
  int idx = INT_MAX;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) argmax_merge(v, idx, x[i], i);
  wave_argmax(v, idx);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = v;
    si[wave] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWavesPerBlock; ++w) argmax_merge(v, idx, sv[w], si[w]);
    store_coherent(pv + blockIdx.x, v);
    store_coherent(pi + blockIdx.x, idx);
    wait_mem();
    const unsigned int prev = arrive(counter);
    s_last = prev == gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last) return;
  v = -INFINITY;
  idx = INT_MAX;
  for (int b = threadIdx.x; b < static_cast<int>(gridDim.x); b += 256)
    argmax_merge(v, idx, load_coherent(pv + b), load_coherent(pi + b));
  wave_argmax(v, idx);
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = v;
    si[wave] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWavesPerBlock; ++w) argmax_merge(v, idx, sv[w], si[w]);
    *out_index = idx;
    *counter = 0u;
  }
}

int argmax_blocks(int n) { return std::max(1, std::min(kArgmaxMaxBlocks, (n + 4095) / 4096)); }

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

const char* kl_error_string(int code) {
  switch (code) {
    case KL_OK: return "ok";
    case KL_EINVAL: return "invalid argument";
    case KL_ENOMEM: return "device out of memory";
    case KL_EFORMAT: return "malformed model image";
    case KL_EUNSUPP: return "unsupported configuration";
    case KL_ETOKEN: return "token id out of range";
    case KL_EWORKSPACE: return "workspace too small";
    case KL_EDEVICE: return "device step error";
    default:
      if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
      return "unknown error";
  }
}

int kl_device_count(int* count) {
  if (!count) return KL_EINVAL;
  return rc(hipGetDeviceCount(count));
}
int kl_set_device(int device) { return rc(hipSetDevice(device)); }
int kl_device_name(int device, char* buf, int buf_len) {
  if (!buf || buf_len <= 0) return KL_EINVAL;
  hipDeviceProp_t prop;
  const hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return rc(e);
  snprintf(buf, buf_len, "%s (%s, %d CUs)", prop.name, prop.gcnArchName, prop.multiProcessorCount);
  return KL_OK;
}
int kl_malloc(void** ptr, size_t bytes) {
  if (!ptr) return KL_EINVAL;
  *ptr = nullptr;
  if (bytes == 0) return KL_OK;
  const hipError_t e = hipMalloc(ptr, bytes);
  if (e == hipErrorOutOfMemory) {
    (void)hipGetLastError();
    return KL_ENOMEM;
  }
  return rc(e);
}
int kl_free(void* ptr) { return ptr ? rc(hipFree(ptr)) : KL_OK; }
int kl_host_alloc(void** ptr, size_t bytes) {
  if (!ptr) return KL_EINVAL;
  return rc(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
}
int kl_host_free(void* ptr) { return ptr ? rc(hipHostFree(ptr)) : KL_OK; }
int kl_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return KL_OK;
  if (!dst || !src) return KL_EINVAL;
  return rc(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
}
int kl_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return KL_OK;
  if (!dst || !src) return KL_EINVAL;
  const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream));
  if (e != hipSuccess) return rc(e);
  return rc(hipStreamSynchronize(as_stream(stream)));
}
int kl_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return KL_OK;
  if (!dst || !src) return KL_EINVAL;
  return rc(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
}
int kl_memset_zero(void* ptr, size_t bytes, void* stream) {
  if (bytes == 0) return KL_OK;
  if (!ptr) return KL_EINVAL;
  return rc(hipMemsetAsync(ptr, 0, bytes, as_stream(stream)));
}
int kl_stream_create(void** stream) {
  if (!stream) return KL_EINVAL;
  hipStream_t s = nullptr;
  const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  *stream = s;
  return rc(e);
}
int kl_stream_destroy(void* stream) { return stream ? rc(hipStreamDestroy(as_stream(stream))) : KL_OK; }
int kl_stream_sync(void* stream) { return rc(hipStreamSynchronize(as_stream(stream))); }
int kl_device_sync(void) { return rc(hipDeviceSynchronize()); }
int kl_event_create(void** event) {
  if (!event) return KL_EINVAL;
  hipEvent_t e = nullptr;
  const hipError_t err = hipEventCreate(&e);
  *event = e;
  return rc(err);
}
int kl_event_destroy(void* event) { return event ? rc(hipEventDestroy(static_cast<hipEvent_t>(event))) : KL_OK; }
int kl_event_record(void* event, void* stream) {
  if (!event) return KL_EINVAL;
  return rc(hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream)));
}
int kl_event_elapsed_ms(void* start, void* stop, float* ms) {
  if (!start || !stop || !ms) return KL_EINVAL;
  const hipError_t e = hipEventSynchronize(static_cast<hipEvent_t>(stop));
  if (e != hipSuccess) return rc(e);
  return rc(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
}

int kl_gemv_f32(const float* x, const float* W, float* y, int rows, int cols, float scale,
                void* stream) {
  if (!x || !W || !y || rows <= 0 || cols <= 0) return KL_EINVAL;
  if (cols % 4 == 0 && aligned16(x) && aligned16(W) && cols <= kMaxKs * 2048) {
    return launch_gemv(x, WView{W, nullptr}, y, rows, cols, false, 0, scale, as_stream(stream));
  } else {
    const int grid = std::max(1, std::min((rows + kWavesPerBlock - 1) / kWavesPerBlock, 4096));
    hipLaunchKernelGGL(k_gemv_f32_scalar, dim3(grid), dim3(256), 0, as_stream(stream), x, W, y,
                       rows, cols, scale);
  }
  return launch_rc();
}

int kl_gemv_q8(const float* x, const int8_t* q, const float* scales, float* y, int rows, int cols,
               int group_size, void* stream) {
  if (!x || !q || !scales || !y || rows <= 0 || cols <= 0 || group_size <= 0) return KL_EINVAL;
  if ((static_cast<int64_t>(rows) * cols) % group_size != 0) return KL_EINVAL;
  const int cpg = group_size / 16;
  const bool vec = group_size % 16 == 0 && (cpg & (cpg - 1)) == 0 && cols % group_size == 0 &&
                   aligned16(x) && aligned16(q) && cols <= kMaxKs * 8192;
  if (vec) {
    return launch_gemv(x, WView{q, scales}, y, rows, cols, true, group_size, 1.f,
                       as_stream(stream));
  } else {
    const int grid = std::max(1, std::min((rows + kWavesPerBlock - 1) / kWavesPerBlock, 4096));
    hipLaunchKernelGGL(k_gemv_q8_scalar, dim3(grid), dim3(256), 0, as_stream(stream), x, q,
                       scales, y, rows, cols, group_size);
  }
  return launch_rc();
}

int kl_dequant_q8(const int8_t* q, const float* scales, int64_t n, int group_size, float* out,
                  void* stream) {
  if (!q || !scales || !out || n <= 0 || group_size <= 0) return KL_EINVAL;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(k_dequant_q8, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     as_stream(stream), q, scales, n, group_size, out);
  return launch_rc();
}

int kl_rmsnorm(const float* x, const float* w, float* y, int n, float eps, void* stream) {
  if (!x || !w || !y || n <= 0) return KL_EINVAL;
  hipLaunchKernelGGL(k_rmsnorm_1, dim3(1), dim3(1024), 0, as_stream(stream), x, w, y, n, eps);
  return launch_rc();
}

int kl_rmsnorm_rows(const float* x, const float* w, float* y, int rows, int n, float eps,
                    void* stream) {
  if (!x || !w || !y || rows <= 0 || n <= 0) return KL_EINVAL;
  if (n <= 4 * kWave * 4 && n % 4 == 0 && aligned16(x) && aligned16(w) && aligned16(y)) {
    const int blocks = (rows + kWavesPerBlock - 1) / kWavesPerBlock;
    hipLaunchKernelGGL(k_rmsnorm_rows_w, dim3(blocks), dim3(256), 0, as_stream(stream), x, w, y,
                       rows, n, eps);
  } else if (n <= 8 * 256 * 4 && n % 4 == 0 && aligned16(x) && aligned16(w) && aligned16(y)) {
    const int r4 = (n / 4 + 255) / 256;  // float4s per thread
    auto launch = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3(rows), dim3(256), 0, as_stream(stream), x, w, y, rows, n, eps);
    };
    if (r4 <= 2) launch(k_rmsnorm_rows_b<2>);
    else if (r4 <= 4) launch(k_rmsnorm_rows_b<4>);
    else launch(k_rmsnorm_rows_b<8>);
  } else {
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(rows), dim3(256), 0, as_stream(stream), x, w, y, rows,
                       n, eps);
  }
  return launch_rc();
}

int kl_sincos_table(int head_size, int seq_len, float theta, float* sin_dev, float* cos_dev) {
  if (head_size <= 0 || seq_len <= 0 || !sin_dev || !cos_dev) return KL_EINVAL;
  const size_t n = static_cast<size_t>(head_size) * seq_len;
  std::vector<float> s(n), c(n);
  for (int pos = 0; pos < seq_len; ++pos) {
    for (int d = 0; d < head_size; ++d) {
      // Same float expression as kernels/cpu/rope_kernel.cpp:7-13.
      const float freq =
          1.0f / std::pow(theta, static_cast<float>(d) / static_cast<float>(head_size));
      const float val = static_cast<float>(pos) * freq;
      s[static_cast<size_t>(pos) * head_size + d] = std::sin(val);
      c[static_cast<size_t>(pos) * head_size + d] = std::cos(val);
    }
  }
  hipError_t e = hipMemcpy(sin_dev, s.data(), n * sizeof(float), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(cos_dev, c.data(), n * sizeof(float), hipMemcpyHostToDevice);
  return rc(e);
}

int kl_rope(int style, int dim, int kv_dim, int head_size, float* q, float* k, int pos,
            const float* sin_cache, const float* cos_cache, void* stream) {
  if (!q || !k || !sin_cache || !cos_cache || dim <= 0 || kv_dim < 0 || kv_dim > dim ||
      head_size <= 0 || head_size % 2 != 0 || dim % head_size != 0 || kv_dim % head_size != 0 ||
      pos < 0)
    return KL_EINVAL;
  if (style != KL_ROPE_INTERLEAVED && style != KL_ROPE_HALF) return KL_EINVAL;
  const int pairs = dim / 2;
  hipLaunchKernelGGL(k_rope, dim3((pairs + 255) / 256), dim3(256), 0, as_stream(stream), style, dim,
                     kv_dim, head_size, q, k, pos, sin_cache, cos_cache);
  return launch_rc();
}

int kl_mha_workspace_size(int head_num, int kv_mul, int seq_len, int head_size, size_t* bytes) {
  if (!bytes || seq_len <= 0 || !mha_shape_ok(head_num, kv_mul, head_size)) return KL_EINVAL;
  size_t need = 0;
  const MhaPlan p = mha_plan_fit(head_num, kv_mul, seq_len, head_size, &need);
  if (p.G > 512) return KL_EUNSUPP;
  *bytes = need;
  return KL_OK;
}

}  // extern "C"

namespace {

// kl_mha's launches with the split partials at `part` (need bytes of the
// mha_plan_fit plan, checked by the caller).
int mha_launch(const MhaPlan& p, int pos, int head_num, int layer_index, int seq_len, int kv_dim,
               int kv_mul, int head_size, float* out, const float* q, float* part,
               const float* key_cache, const float* value_cache, hipStream_t st) {
  const int kv_heads = head_num / kv_mul;
  AttnArgs a{};
  const size_t layer_off = static_cast<size_t>(layer_index) * seq_len * kv_dim;
  a.q = q;
  a.kcache = const_cast<float*>(key_cache) + layer_off;
  a.vcache = value_cache + layer_off;
  a.out = out;
  a.part = part;
  a.counters = nullptr;  // the spans are merged by k_attn_merge: no counter to initialise
  a.pos_ptr = nullptr;
  a.pos_val = pos;
  a.kv_dim = kv_dim;
  a.kv_mul = kv_mul;
  a.G = p.G;
  a.cpw = p.cpw;
  a.transform = 0;
  a.scale = 1.f / std::sqrt(static_cast<float>(head_size));
  const int span = attn_chunk(head_size) * p.cpw;
  const int nsplit = (pos + span) / span;
  const dim3 grid(kv_heads * p.G), block(256);
  const size_t merge_lds = static_cast<size_t>(nsplit) * kv_mul * 2 * sizeof(float);
  switch (head_size) {
    case 32: hipLaunchKernelGGL(k_attn_decode<32>, grid, block, p.lds_bytes, st, a); break;
    case 64: hipLaunchKernelGGL(k_attn_decode<64>, grid, block, p.lds_bytes, st, a); break;
    case 128: hipLaunchKernelGGL(k_attn_decode<128>, grid, block, p.lds_bytes, st, a); break;
    default: hipLaunchKernelGGL(k_attn_decode<256>, grid, block, p.lds_bytes, st, a); break;
  }
  if (nsplit > 1) {
    const dim3 mg(kv_heads);
    switch (head_size) {
      case 32: hipLaunchKernelGGL(k_attn_merge<32>, mg, block, merge_lds, st, a); break;
      case 64: hipLaunchKernelGGL(k_attn_merge<64>, mg, block, merge_lds, st, a); break;
      case 128: hipLaunchKernelGGL(k_attn_merge<128>, mg, block, merge_lds, st, a); break;
      default: hipLaunchKernelGGL(k_attn_merge<256>, mg, block, merge_lds, st, a); break;
    }
  }
  return launch_rc();
}

// Argument checks shared by kl_mha and kl_mha_noalloc; on success *p is the
// plan and *need its workspace bytes.
int mha_check(int pos, int head_num, int layer_index, int seq_len, int kv_dim, int kv_mul,
              int head_size, const float* out, const float* q, const float* key_cache,
              const float* value_cache, MhaPlan* p, size_t* need) {
  if (!out || !q || !key_cache || !value_cache) return KL_EINVAL;
  if (!mha_shape_ok(head_num, kv_mul, head_size)) return KL_EUNSUPP;
  if (pos < 0 || pos >= seq_len || layer_index < 0) return KL_EINVAL;
  if (kv_dim != head_num / kv_mul * head_size) return KL_EINVAL;
  *p = mha_plan_fit(head_num, kv_mul, seq_len, head_size, need);
  if (p->G > 512) return KL_EUNSUPP;
  return KL_OK;
}

// The no-allocation variant's partials: one array per device, found with
// hipGetSymbolAddress on the first call on each device (the array's host-side
// name is not a device address).
constexpr size_t kMhaScratchBytes = size_t(1) << 20;
static __device__ __align__(256) unsigned char scratch[kMhaScratchBytes];
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

int scratch_for_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return rc(e);
  if (dev < 0 || dev >= kMaxScratchDevices) return KL_EUNSUPP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return rc(e);
    if (!p) return KL_EDEVICE;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KL_OK;
}

}  // namespace

extern "C" {

int kl_mha(int pos, int head_num, int layer_index, int seq_len, int kv_dim, int kv_mul,
           int head_size, float* out, const float* q, void* workspace, size_t workspace_bytes,
           const float* key_cache, const float* value_cache, void* stream) {
  if (!workspace) return KL_EINVAL;
  MhaPlan p;
  size_t need = 0;
  const int r = mha_check(pos, head_num, layer_index, seq_len, kv_dim, kv_mul, head_size, out, q,
                          key_cache, value_cache, &p, &need);
  if (r != KL_OK) return r;
  if (workspace_bytes < need) return KL_EWORKSPACE;
  return mha_launch(p, pos, head_num, layer_index, seq_len, kv_dim, kv_mul, head_size, out, q,
                    static_cast<float*>(workspace), key_cache, value_cache, as_stream(stream));
}

size_t kl_mha_noalloc_max_bytes(void) { return kMhaScratchBytes; }

int kl_mha_noalloc(int pos, int head_num, int layer_index, int seq_len, int kv_dim, int kv_mul,
                   int head_size, float* out, const float* q, const float* key_cache,
                   const float* value_cache, void* stream) {
  MhaPlan p;
  size_t need = 0;
  int r = mha_check(pos, head_num, layer_index, seq_len, kv_dim, kv_mul, head_size, out, q,
                    key_cache, value_cache, &p, &need);
  if (r != KL_OK) return r;
  if (need > kMhaScratchBytes) return KL_EWORKSPACE;
  void* part = nullptr;
  r = scratch_for_current_device(&part);
  if (r != KL_OK) return r;
  return mha_launch(p, pos, head_num, layer_index, seq_len, kv_dim, kv_mul, head_size, out, q,
                    static_cast<float*>(part), key_cache, value_cache, as_stream(stream));
}

int kl_qk_norm_rope_rows(int style, int head_size, int q_heads, int kv_heads, float* q, int ldq,
                         float* k, int ldk, const float* q_norm, const float* k_norm, float eps,
                         int pos0, int n_pos, const float* sin_cache, const float* cos_cache,
                         void* stream) {
  if (!q || !k || !q_norm || !k_norm || !sin_cache || !cos_cache || q_heads <= 0 ||
      kv_heads <= 0 || pos0 < 0 || n_pos <= 0 || ldq < q_heads * head_size ||
      ldk < kv_heads * head_size)
    return KL_EINVAL;
  if (style != KL_ROPE_INTERLEAVED && style != KL_ROPE_HALF) return KL_EINVAL;
  if (head_size != 64 && head_size != 128) return KL_EUNSUPP;
  if (ldq % 4 || ldk % 4 || !aligned16(q) || !aligned16(k) || !aligned16(q_norm) ||
      !aligned16(k_norm) || !aligned16(sin_cache) || !aligned16(cos_cache))
    return KL_EUNSUPP;
  const long long groups = static_cast<long long>(n_pos) * (q_heads + kv_heads);
  const long long waves = (groups + kWave / (head_size / 4) - 1) / (kWave / (head_size / 4));
  const long long blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  if (blocks > INT_MAX) return KL_EINVAL;
  if (head_size == 128)
    hipLaunchKernelGGL(k_qk_norm_rope_rows<128>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       as_stream(stream), style, q_heads, kv_heads, q, ldq, k, ldk, q_norm, k_norm,
                       eps, pos0, n_pos, sin_cache, cos_cache);
  else
    hipLaunchKernelGGL(k_qk_norm_rope_rows<64>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       as_stream(stream), style, q_heads, kv_heads, q, ldq, k, ldk, q_norm, k_norm,
                       eps, pos0, n_pos, sin_cache, cos_cache);
  return launch_rc();
}

int kl_rope_rows(int style, int dim, int kv_dim, int head_size, float* q, int ldq, float* k,
                 int ldk, int pos0, int n_pos, const float* sin_cache, const float* cos_cache,
                 void* stream) {
  if (!q || !k || !sin_cache || !cos_cache || dim <= 0 || kv_dim < 0 || kv_dim > dim ||
      head_size <= 0 || head_size % 2 != 0 || dim % head_size != 0 || kv_dim % head_size != 0 ||
      pos0 < 0 || n_pos <= 0 || n_pos > 65535 || ldq < dim || ldk < kv_dim)
    return KL_EINVAL;
  if (style != KL_ROPE_INTERLEAVED && style != KL_ROPE_HALF) return KL_EINVAL;
  const int pairs = dim / 2;
  hipLaunchKernelGGL(k_rope_rows, dim3((pairs + 255) / 256, n_pos), dim3(256), 0, as_stream(stream),
                     style, dim, kv_dim, head_size, q, ldq, k, ldk, pos0, n_pos, sin_cache,
                     cos_cache);
  return launch_rc();
}

}  // extern "C"

namespace {
constexpr int kGemmTile = 64;  // workgroup tile of both GEMM kernels (2 x 2 waves of 32 x 32)

bool gemm_shape_ok(const float* A, int M, int K, int lda) {
  return A && M > 0 && K > 0 && lda >= K;
}

}  // namespace

// C_s (+)= A . W_s^T (+ bias_s) for nseg outputs in one grid; splits > 1
// (nseg == 1) divides K among blockIdx.y into ws[splits][M][N] and reduces.
int kl::gemm_run(const float* A, int M, int K, int lda, int nseg, const GemmSeg* segs,
                 int accumulate, float* ws, int splits, hipStream_t st) {
  if (!gemm_shape_ok(A, M, K, lda) || nseg < 1 || nseg > kGemmMaxSeg || splits < 1 ||
      (splits > 1 && !ws))
    return KL_EINVAL;
  if (K % 4 || lda % 4 || !aligned16(A)) return KL_EUNSUPP;
  // The kernel addresses each operand with 32-bit byte offsets.
  if (static_cast<size_t>(M) * lda * sizeof(float) > 0xFFFFFFFFu) return KL_EUNSUPP;
  const bool q8 = segs[0].S != nullptr;
  if (q8) {
    // int8: whole K blocks, the image's dense rows (ldw == K), 4-byte loads.
    if (K % kGemmBK) return KL_EUNSUPP;
    for (int i = 0; i < nseg; ++i) {
      const GemmSeg& sg = segs[i];
      if (!sg.S || sg.ldw != K || (reinterpret_cast<uintptr_t>(sg.W) & 3u) || sg.gshift < 2 ||
          sg.gshift > 20)
        return KL_EUNSUPP;
      if (!sg.W || !sg.C || sg.N <= 0 || sg.ldc < sg.N) return KL_EINVAL;
      if (static_cast<size_t>(sg.N) * sg.ldw > 0xFFFFFFFFu) return KL_EUNSUPP;
    }
  }
  GemmArgs g{};
  g.A = A;
  g.M = M;
  g.K = K;
  g.lda = lda;
  g.accumulate = accumulate;
  g.nseg = nseg;
  g.ws = ws;
  g.splits = splits;
  // int8 weights with at most 32 rows: 32 x 128 tiles (no padded rows).
  // fp32 through the direct-to-LDS kernel: 128 x 64 tiles where the launch
  // has at least 1024 of them (two rounds of two workgroups per CU), else
  // 64 x 64.
  const bool small = q8 && M <= 32;
  const bool dma = !q8 && K % kGemmBK == 0;
  bool tall = false;
  if (dma && M >= 128) {
    long long t = 0;
    for (int i = 0; i < nseg; ++i) t += static_cast<long long>((M + 127) / 128) * ((segs[i].N + 63) / 64);
    tall = t >= 1024;
  }
  const int bm = small ? 32 : tall ? 128 : kGemmTile, bn = small ? 128 : kGemmTile;
  g.tiles_m = (M + bm - 1) / bm;
  long long tiles = 0;
  size_t wsoff = 0;
  for (int i = 0; i < nseg; ++i) {
    const GemmSeg& sg = segs[i];
    if (!q8) {
      if (sg.S || !sg.W || !sg.C || sg.N <= 0 || sg.ldw < K || sg.ldc < sg.N) return KL_EINVAL;
      if (sg.ldw % 4 || !aligned16(sg.W)) return KL_EUNSUPP;
      if (static_cast<size_t>(sg.N) * sg.ldw * sizeof(float) > 0xFFFFFFFFu) return KL_EUNSUPP;
    }
    g.seg[i] = sg;
    g.seg[i].tile0 = static_cast<int>(tiles);
    g.seg[i].wsoff = wsoff;
    tiles += static_cast<long long>(g.tiles_m) * ((sg.N + bn - 1) / bn);
    wsoff += static_cast<size_t>(M) * sg.N;
  }
  g.ws_split = wsoff;
  if (tiles > INT_MAX) return KL_EUNSUPP;
  // fp32 weights with K a whole number of 32-column blocks (every model
  // projection) stream through the direct-to-LDS kernel; int8 weights and
  // other K through the register-staged one.
  // Short int8 prompts with groups of at least 32 (one scale per row and
  // 32-column block) and 16-byte aligned weights stage the int8 tiles
  // directly into LDS.
  bool small_dma = small;
  for (int i = 0; i < nseg && small_dma; ++i)
    small_dma = segs[i].gshift >= 5 && (reinterpret_cast<uintptr_t>(segs[i].W) & 15u) == 0;
  if (small_dma)
    hipLaunchKernelGGL(k_gemm_q8_dma, dim3(static_cast<unsigned>(tiles), splits), dim3(256), 0, st, g);
  else if (small)
    hipLaunchKernelGGL((k_gemm_f32<1, 4, 1, 1, true>), dim3(static_cast<unsigned>(tiles), splits),
                       dim3(256), 0, st, g);
  else if (q8)
    hipLaunchKernelGGL((k_gemm_f32<2, 2, 1, 1, true>), dim3(static_cast<unsigned>(tiles), splits),
                       dim3(256), 0, st, g);
  else if (tall)
    hipLaunchKernelGGL(k_gemm_f32_dma<4>, dim3(static_cast<unsigned>(tiles), splits), dim3(256), 0, st, g);
  else if (dma)
    hipLaunchKernelGGL(k_gemm_f32_dma<2>, dim3(static_cast<unsigned>(tiles), splits), dim3(256), 0, st, g);
  else
    hipLaunchKernelGGL((k_gemm_f32<2, 2, 1, 1>), dim3(static_cast<unsigned>(tiles), splits), dim3(256),
                       0, st, g);
  int r = launch_rc();
  if (r != KL_OK || splits == 1) return r;
  const int grid = static_cast<int>(std::min<size_t>((g.ws_split + 255) / 256, 4096));
  hipLaunchKernelGGL(k_gemm_reduce, dim3(grid), dim3(256), 0, st, g);
  return launch_rc();
}

extern "C" {

int kl_gemm_f32(const float* A, const float* W, float* C, int M, int N, int K, int lda, int ldw,
                int ldc, const float* bias, int accumulate, void* stream) {
  if (!gemm_shape_ok(A, M, K, lda) || !W || !C || N <= 0 || ldw < K || ldc < N) return KL_EINVAL;
  const GemmSeg sg{W, C, bias, N, ldw, ldc, 0};
  return gemm_run(A, M, K, lda, 1, &sg, accumulate, nullptr, 1, as_stream(stream));
}

int kl_gemm_f32_grouped(const float* A, int M, int K, int lda, int n_seg, const float* const* W,
                        float* const* C, const float* const* bias, const int* N, const int* ldw,
                        const int* ldc, int accumulate, void* stream) {
  if (!gemm_shape_ok(A, M, K, lda) || n_seg < 1 || n_seg > kGemmMaxSeg || !W || !C || !N || !ldw ||
      !ldc)
    return KL_EINVAL;
  GemmSeg segs[kGemmMaxSeg];
  for (int i = 0; i < n_seg; ++i)
    segs[i] = GemmSeg{W[i], C[i], bias ? bias[i] : nullptr, N[i], ldw[i], ldc[i], 0};
  return gemm_run(A, M, K, lda, n_seg, segs, accumulate, nullptr, 1, as_stream(stream));
}

int kl_gemm_q8(const float* A, const int8_t* q, const float* scales, int group_size, float* C,
               int M, int N, int K, int lda, int ldc, const float* bias, int accumulate, int splits,
               void* workspace, size_t workspace_bytes, void* stream) {
  if (!gemm_shape_ok(A, M, K, lda) || !q || !scales || !C || N <= 0 || ldc < N || splits < 1 ||
      splits > 16 || group_size < 4 || (group_size & (group_size - 1)))
    return KL_EINVAL;
  if (splits > 1 && (!workspace || workspace_bytes < static_cast<size_t>(splits) * M * N * sizeof(float)))
    return KL_EWORKSPACE;
  int gshift = 0;
  while ((1 << gshift) < group_size) ++gshift;
  GemmSeg sg{q, C, bias, N, K, ldc, 0, scales, gshift};
  return gemm_run(A, M, K, lda, 1, &sg, accumulate, static_cast<float*>(workspace), splits,
                  as_stream(stream));
}

int kl_gemm_f32_splitk(const float* A, const float* W, float* C, int M, int N, int K, int lda,
                       int ldw, int ldc, const float* bias, int accumulate, int splits,
                       void* workspace, size_t workspace_bytes, void* stream) {
  if (!gemm_shape_ok(A, M, K, lda) || !W || !C || N <= 0 || ldw < K || ldc < N || splits < 1 ||
      splits > 16)
    return KL_EINVAL;
  if (splits > 1 && (!workspace || workspace_bytes < static_cast<size_t>(splits) * M * N * sizeof(float)))
    return KL_EWORKSPACE;
  const GemmSeg sg{W, C, bias, N, ldw, ldc, 0};
  return gemm_run(A, M, K, lda, 1, &sg, accumulate, static_cast<float*>(workspace), splits,
                     as_stream(stream));
}

}  // extern "C"

namespace {
int device_cus();

// Time model of k_gemm_x6 launches, one workgroup per CU: rounds of the grid
// x 32-column blocks per split x the block time of the tile (1.45 us for 128
// x 128, 2.3 us for 256 x 128: measured on the Qwen3-4B and Qwen2.5-1.5B
// shapes), plus (splits > 1) the partials written and read once and the
// outputs written ((2 splits + 1) x mn floats) at 4 TB/s.
double x6_time(long long units, int kblocks, size_t mn, int splits, double blk) {
  const long long cus = device_cus();
  return static_cast<double>((units + cus - 1) / cus) * kblocks * blk +
         (splits > 1 ? static_cast<double>(mn) * 4.0 * (2 * splits + 1) / 4e6 : 0.0);
}

// The split count (1 .. 8, each split at least 4 blocks, partials within
// ws_floats) with the least modelled time; a larger count must win by 3%.
int x6_splits(long long tiles, int nkt, size_t mn, size_t ws_floats, double blk, double* t_out) {
  int best = 1;
  double tbest = 1e300;
  for (int s = 1; s <= 8 && nkt / s >= 4; ++s) {
    if (s > 1 && static_cast<size_t>(s) * mn > ws_floats) break;
    const double t = x6_time(tiles * s, (nkt + s - 1) / s, mn, s, blk);
    if (t < tbest * 0.97) {
      tbest = t;
      best = s;
    }
  }
  if (t_out) *t_out = tbest;
  return best;
}

template <int WMW, int NPW>
int x6_launch(GemmX6Args x, int splits, hipStream_t st) {
  const unsigned grid = static_cast<unsigned>(8 * ((x.tiles + 7) / 8));
  hipLaunchKernelGGL((k_gemm_x6<WMW, NPW>), dim3(grid, splits), dim3(128 * WMW), 0, st, x);
  return launch_rc();
}
}  // namespace

int kl::gemm_run_x6(const GemmX6Planes& planes, int M, int K, int nseg, const GemmSeg* segs,
                    int accumulate, float* ws, size_t ws_bytes, hipStream_t st, int* deferred) {
  if (!planes.A || M <= 0 || K <= 0 || nseg < 1 || nseg > kGemmMaxSeg) return KL_EINVAL;
  if (K % 32 || !aligned16(planes.A)) return KL_EUNSUPP;
  for (int i = 0; i < nseg; ++i) {
    const GemmSeg& sg = segs[i];
    if (!planes.W[i] || !sg.C || sg.N <= 0 || sg.ldc < sg.N || sg.S) return KL_EINVAL;
    if (!aligned16(planes.W[i])) return KL_EUNSUPP;
  }
  // Tile: 256 x 128 from 256 rows (KL_X6_TILE=128 keeps 128 x 128).
  static const int force128 = [] {
    const char* e = std::getenv("KL_X6_TILE");
    return e && std::atoi(e) == 128;
  }();
  const int wmw = M >= 256 && !force128 ? 4 : 2;
  // W planes (1: bf16-exact weights).  The split and tail choice ignores it,
  // so both forms sum in the same order and give the same values.
  const int npw = planes.w_planes == 1 ? 1 : 3;
  const int bm = 64 * wmw;
  const double blk = wmw == 4 ? 2.3 : 1.45;
  const int nkt = K / 32;
  const size_t ws_floats = ws ? ws_bytes / sizeof(float) : 0;
  auto build = [&](GemmX6Args& x, int n, const GemmSeg* sgs, const void* const* W) {
    GemmArgs g{};
    g.M = M;
    g.K = K;
    g.accumulate = accumulate;
    g.nseg = n;
    g.ws = ws;
    g.tiles_m = (M + bm - 1) / bm;
    x = GemmX6Args{};
    x.p.A = planes.A;
    long long tiles = 0;
    size_t wsoff = 0;
    for (int i = 0; i < n; ++i) {
      x.p.W[i] = W[i];
      g.seg[i] = sgs[i];
      g.seg[i].tile0 = static_cast<int>(tiles);
      g.seg[i].wsoff = wsoff;
      tiles += static_cast<long long>(g.tiles_m) * ((sgs[i].N + 127) / 128);
      wsoff += static_cast<size_t>(M) * sgs[i].N;
    }
    g.ws_split = wsoff;
    x.g = g;
    x.tiles = static_cast<int>(std::min<long long>(tiles, INT_MAX));
    return tiles;
  };
  auto run = [&](GemmX6Args& x, int splits, bool reduce) {
    x.g.splits = splits;
    int r = wmw == 4 ? (npw == 1 ? x6_launch<4, 1>(x, splits, st) : x6_launch<4, 3>(x, splits, st))
                     : (npw == 1 ? x6_launch<2, 1>(x, splits, st) : x6_launch<2, 3>(x, splits, st));
    if (r != KL_OK || splits == 1 || !reduce) return r;
    const int rgrid = static_cast<int>(std::min<size_t>((x.g.ws_split + 255) / 256, 4096));
    hipLaunchKernelGGL(k_gemm_reduce, dim3(rgrid), dim3(256), 0, st, x.g);
    return launch_rc();
  };
  GemmX6Args x;
  const long long tiles = build(x, nseg, segs, planes.W);
  if (tiles > INT_MAX / 2) return KL_EUNSUPP;
  const size_t mn = x.g.ws_split;
  double t_plain = 0;
  const int sp = ws ? x6_splits(tiles, nkt, mn, ws_floats, blk, &t_plain) : 1;
  // Whole rounds plus a split-K tail: the tail is the last tail_tiles tiles
  // (whole tile columns of the last output), split to fill the CUs.
  const long long cus = device_cus();
  const int tm = x.g.tiles_m;
  const GemmSeg& last = segs[nseg - 1];
  const long long last_cols = (last.N + 127) / 128;
  long long tail_cols = (tiles % cus + tm - 1) / tm;
  if (ws && tiles > cus && tail_cols > 0 && tail_cols < last_cols) {
    const long long tail = tail_cols * tm, main = tiles - tail;
    const size_t tmn = static_cast<size_t>(M) * (last.N - (last_cols - tail_cols) * 128);
    double t_tail = 0;
    const int tsp = x6_splits(tail, nkt, tmn, ws_floats, blk, &t_tail);
    const double t_split = x6_time(main, nkt, 0, 1, blk) + t_tail;
    if (t_split < t_plain * 0.97) {
      const int c0 = static_cast<int>((last_cols - tail_cols) * 128);
      GemmSeg hs[kGemmMaxSeg];
      const void* hw[kGemmMaxSeg];
      for (int i = 0; i < nseg; ++i) {
        hs[i] = segs[i];
        hw[i] = planes.W[i];
      }
      hs[nseg - 1].N = c0;  // main: the last output's first c0 columns
      GemmX6Args xm;
      build(xm, nseg, hs, hw);
      int r = run(xm, 1, true);
      // tail: columns c0 .. N of the last output (its W planes from row c0)
      GemmSeg ts = last;
      ts.C = last.C + c0;
      if (ts.bias) ts.bias = last.bias + c0;
      ts.N = last.N - c0;
      const void* tw = static_cast<const char*>(planes.W[nseg - 1]) +
                       static_cast<size_t>(c0 / 16) * (K / 32) * 1536 * sizeof(__bf16);
      GemmX6Args xt;
      build(xt, 1, &ts, &tw);
      if (r == KL_OK) r = run(xt, tsp, true);
      if (deferred) *deferred = 1;
      return r;
    }
  }
  if (deferred) *deferred = sp;
  return run(x, sp, !deferred);
}

namespace {
// Split count of a k_gemm_q8s launch of `wgs` workgroups over ng groups of
// cpg chunks and mn output floats, one workgroup per CU: rounds x (3 us +
// 1.2 us per group of a split) plus the partials written and read once
// ((2 splits + 1) mn floats at 4 TB/s); a split's activations must fit the
// kernel's LDS (kQ8sLdsChunks chunks), and a split count must win by 3% over
// the next smaller one.  0 when no split count up to 64 fits.
int q8s_splits(long long wgs, int ng, int cpg, size_t mn, size_t ws_floats) {
  const long long slots = device_cus();
  int best = 0;
  double tbest = 1e300;
  for (int s = 1; s <= 64 && s <= ng; ++s) {
    if ((ng + s - 1) / s * cpg > kQ8sLdsChunks) continue;
    if (s > 1 && static_cast<size_t>(s) * mn > ws_floats) break;
    const long long rounds = (wgs * s + slots - 1) / slots;
    const double t = static_cast<double>(rounds) * (3.0 + ((ng + s - 1) / s) * 1.2) +
                     (s > 1 ? static_cast<double>(mn) * 4.0 * (2 * s + 1) / 4e6 : 0.0);
    if (t < tbest * 0.97) {
      tbest = t;
      best = s;
    }
  }
  return best;
}

bool q8s_group_ok(int K, int group_size) {
  return (group_size == 32 || group_size == 64) && K > 0 && K % group_size == 0;
}
}  // namespace

size_t kl::q8s_packed_bytes(int N, int K, int group_size) {
  if (N <= 0 || !q8s_group_ok(K, group_size)) return 0;
  return q8s_tile_bytes(N, K) + static_cast<size_t>((N + 31) / 32) * (K / group_size) * 32 * sizeof(float);
}

int kl::q8s_pack_run(const int8_t* q, const float* scales, int N, int K, int group_size, void* packed,
                     hipStream_t st) {
  if (!q || !scales || !packed || N <= 0) return KL_EINVAL;
  if (!q8s_group_ok(K, group_size) || !aligned16(q) || !aligned16(packed)) return KL_EUNSUPP;
  int gshift = 0;
  while ((1 << gshift) < group_size) ++gshift;
  const size_t work = static_cast<size_t>((N + 31) / 32) * (K / 32) * 64 +
                      static_cast<size_t>((N + 31) / 32) * (K / group_size) * 32;
  const int grid = static_cast<int>(std::min<size_t>((work + 255) / 256, 16384));
  hipLaunchKernelGGL(k_q8s_pack, dim3(grid), dim3(256), 0, st, q, scales, N, K, gshift,
                     static_cast<char*>(packed));
  return launch_rc();
}

int kl::q8s_split_run(const float* A, int M, int K, int lda, void* planes, hipStream_t st) {
  if (!A || !planes || M <= 0 || M > 32 || K <= 0 || lda < K) return KL_EINVAL;
  if (K % 32 || lda % 4 || !aligned16(A) || !aligned16(planes)) return KL_EUNSUPP;
  const size_t work = static_cast<size_t>(K / 32) * 128;
  const int grid = static_cast<int>(std::min<size_t>((work + 255) / 256, 4096));
  hipLaunchKernelGGL(k_q8s_split, dim3(grid), dim3(256), 0, st, A, M, K, lda, static_cast<__bf16*>(planes));
  return launch_rc();
}

int kl::gemm_run_q8s(const void* planes, int M, int K, int group_size, int nseg, const GemmSeg* segs,
                     int accumulate, float* ws, size_t ws_bytes, hipStream_t st, int* deferred) {
  if (!planes || M <= 0 || M > 32 || nseg < 1 || nseg > kGemmMaxSeg) return KL_EINVAL;
  if (!q8s_group_ok(K, group_size) || !aligned16(planes)) return KL_EUNSUPP;
  GemmQ8sArgs g{};
  g.A = planes;
  g.M = M;
  g.K = K;
  while ((1 << g.gshift) < group_size) ++g.gshift;
  g.accumulate = accumulate;
  g.nseg = nseg;
  g.ws = ws;
  long long wgs = 0;
  size_t wsoff = 0;
  for (int i = 0; i < nseg; ++i) {
    const GemmSeg& sg = segs[i];
    if (!sg.W || !sg.C || sg.N <= 0 || sg.ldc < sg.N) return KL_EINVAL;
    if (!aligned16(sg.W)) return KL_EUNSUPP;
    g.seg[i] = GemmQ8sSeg{sg.W, sg.C, sg.bias, sg.N, sg.ldc, static_cast<int>(wgs), wsoff};
    wgs += (sg.N + 511) / 512;
    wsoff += static_cast<size_t>(M) * sg.N;
  }
  if (wgs > INT_MAX / 2) return KL_EUNSUPP;
  g.ws_split = wsoff;
  g.splits = q8s_splits(wgs, K / group_size, group_size / 32, wsoff, ws ? ws_bytes / sizeof(float) : 0);
  if (g.splits == 0) return KL_EWORKSPACE;  // K too deep for one split's LDS: room for partials needed
  const dim3 grid(static_cast<unsigned>(wgs), g.splits);
  if (group_size == 32)
    hipLaunchKernelGGL(k_gemm_q8s<1>, grid, dim3(512), 0, st, g);
  else
    hipLaunchKernelGGL(k_gemm_q8s<2>, grid, dim3(512), 0, st, g);
  int r = launch_rc();
  if (deferred) *deferred = g.splits;
  if (r != KL_OK || g.splits == 1 || deferred) return r;
  // k_gemm_reduce reads the output list of a GemmArgs.
  GemmArgs ra{};
  ra.M = M;
  ra.accumulate = accumulate;
  ra.nseg = nseg;
  ra.ws = ws;
  ra.ws_split = wsoff;
  ra.splits = g.splits;
  for (int i = 0; i < nseg; ++i) {
    ra.seg[i].C = segs[i].C;
    ra.seg[i].bias = segs[i].bias;
    ra.seg[i].N = segs[i].N;
    ra.seg[i].ldc = segs[i].ldc;
    ra.seg[i].wsoff = g.seg[i].wsoff;
  }
  const int rgrid = static_cast<int>(std::min<size_t>((wsoff + 255) / 256, 4096));
  hipLaunchKernelGGL(k_gemm_reduce, dim3(rgrid), dim3(256), 0, st, ra);
  return launch_rc();
}

// RMSNorm of one row per workgroup into GEMM-input planes (the arithmetic
// of k_rmsnorm_rows_b), after x += the row's split-K partials summed in split
// order (the arithmetic of k_gemm_reduce with accumulate), written back.
// With gridDim.y > 1 (no partials), workgroup (row, c) computes the row's
// norm the same way and stores float4 columns [c, c + 1) n4 / gridDim.y only,
// so that a few rows still spread over many CUs (same bits).
template <int R>
__global__ __launch_bounds__(256) void k_norm_planes(float* x, const float* __restrict__ w, int n,
                                                     float eps, const float* __restrict__ ws,
                                                     int splits, size_t ws_split, __bf16* planes,
                                                     bool q8s) {
  __shared__ float red[kWavesPerBlock];
  const int row = blockIdx.x;
  f4* xr = reinterpret_cast<f4*>(x + static_cast<size_t>(row) * n);
  const f4* w4 = reinterpret_cast<const f4*>(w);
  const int n4 = n / 4;
  f4 v[R];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int i = threadIdx.x + j * 256;
    v[j] = f4{0.f, 0.f, 0.f, 0.f};
    if (i < n4) {
      v[j] = xr[i];
      if (splits > 0) {
        const f4* p = reinterpret_cast<const f4*>(ws + static_cast<size_t>(row) * n) + i;
        v[j] = v[j] + split_sum(p, ws_split / 4, splits);
        xr[i] = v[j];
      }
    }
    ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
  }
  ss = block_sum(ss, red);
  const float r = 1.f / sqrtf(ss / static_cast<float>(n) + eps);
  const int c0 = static_cast<int>(blockIdx.y * static_cast<long long>(n4) / gridDim.y);
  const int c1 = static_cast<int>((blockIdx.y + 1) * static_cast<long long>(n4) / gridDim.y);
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int i = threadIdx.x + j * 256;
    if (i >= c0 && i < c1) planes_store4(q8s, planes, row, 4 * i, n, (r * v[j]) * w4[i]);
  }
}

// silu(h1) * h3 (the arithmetic of k_swiglu) into GEMM-input planes, h1 and
// h3 summed from split-K partials in split order when splits > 0.
__global__ void k_swiglu_planes(const float* __restrict__ h1, const float* __restrict__ h3, int rows,
                                int F, const float* __restrict__ ws, int splits, size_t ws_split,
                                size_t wsoff3, __bf16* planes, bool q8s) {
  const int f4n = F / 4;
  const size_t total = static_cast<size_t>(rows) * f4n;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int r = static_cast<int>(i / f4n), c = static_cast<int>(i - static_cast<size_t>(r) * f4n) * 4;
    const size_t o = static_cast<size_t>(r) * F + c;
    f4 a, b;
    if (splits > 0) {
      a = split_sum(reinterpret_cast<const f4*>(ws + o), ws_split / 4, splits);
      b = split_sum(reinterpret_cast<const f4*>(ws + wsoff3 + o), ws_split / 4, splits);
    } else {
      a = *reinterpret_cast<const f4*>(h1 + o);
      b = *reinterpret_cast<const f4*>(h3 + o);
    }
    f4 out;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float av = a[e];
      const float sl = av * (1.0f / (1.0f + expf(-av)));
      out[e] = sl * b[e];
    }
    planes_store4(q8s, planes, r, c, F, out);
  }
}

// q, k and v of a grouped Q/K/V launch summed from its split-K partials
// (ws + z ws_split, segments at 0, n dim and n (dim + kv_dim), rows of dim /
// kv_dim / kv_dim), in split order plus the bias -- k_gemm_reduce's
// arithmetic -- then q and k rotated as k_rope_rows rotates them, and all
// three stored: one pass in place of the reduction and the rotation (same
// bits).  Thread p of row r owns q's pair p, k's pair p where rope_one
// rotates it (which covers every k element), and v elements 2p, 2p + 1.
__global__ void k_qkv_sum_rope_rows(int style, int dim, int kv_dim, int hd, const float* __restrict__ ws,
                                    int splits, size_t ws_split, const float* __restrict__ bq,
                                    const float* __restrict__ bk, const float* __restrict__ bv, float* q,
                                    int ldq, float* k, int ldk, float* v, int ldv, int pos0, int n,
                                    const float* __restrict__ sin_t, const float* __restrict__ cos_t) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  const int r = blockIdx.y;
  if (p >= dim / 2 || r >= n) return;
  int i0, i1, tab;
  rope_index(style, hd, p, i0, i1, tab);
  const int pos = pos0 + r;
  const float fci = sin_t[static_cast<size_t>(pos) * hd + tab];
  const float fcr = cos_t[static_cast<size_t>(pos) * hd + tab];
  const float* pq = ws + static_cast<size_t>(r) * dim;
  float v0 = split_sum(pq + i0, ws_split, splits), v1 = split_sum(pq + i1, ws_split, splits);
  if (bq) {
    v0 += bq[i0];
    v1 += bq[i1];
  }
  rope_pair(v0, v1, fcr, fci);
  float* qr = q + static_cast<size_t>(r) * ldq;
  qr[i0] = v0;
  qr[i1] = v1;
  const int gate = style == KL_ROPE_INTERLEAVED ? i0 : (i0 - (i0 % hd));
  if (gate < kv_dim) {
    const float* pk = ws + static_cast<size_t>(n) * dim + static_cast<size_t>(r) * kv_dim;
    float w0 = split_sum(pk + i0, ws_split, splits), w1 = split_sum(pk + i1, ws_split, splits);
    if (bk) {
      w0 += bk[i0];
      w1 += bk[i1];
    }
    rope_pair(w0, w1, fcr, fci);
    float* kr = k + static_cast<size_t>(r) * ldk;
    kr[i0] = w0;
    kr[i1] = w1;
  }
  if (2 * p < kv_dim) {
    const float* pv = ws + static_cast<size_t>(n) * (dim + kv_dim) + static_cast<size_t>(r) * kv_dim;
    float* vr = v + static_cast<size_t>(r) * ldv;
#pragma unroll
    for (int e = 2 * p; e < 2 * p + 2; ++e) {
      float x = split_sum(pv + e, ws_split, splits);
      if (bv) x += bv[e];
      vr[e] = x;
    }
  }
}

int kl::qkv_sum_rope_run(int style, int dim, int kv_dim, int hd, const float* ws, int splits,
                         size_t ws_split, const float* bq, const float* bk, const float* bv, float* q,
                         int ldq, float* k, int ldk, float* v, int ldv, int pos0, int n,
                         const float* sin_t, const float* cos_t, hipStream_t st) {
  if (!ws || !q || !k || !v || !sin_t || !cos_t || splits < 1 || n <= 0 || n > 65535 || pos0 < 0 ||
      hd <= 0 || hd % 2 || dim <= 0 || kv_dim <= 0 || kv_dim > dim || dim % hd || kv_dim % hd ||
      ldq < dim || ldk < kv_dim || ldv < kv_dim ||
      ws_split < static_cast<size_t>(n) * (dim + 2 * static_cast<size_t>(kv_dim)))
    return KL_EINVAL;
  if (style != KL_ROPE_INTERLEAVED && style != KL_ROPE_HALF) return KL_EINVAL;
  const int pairs = dim / 2;
  hipLaunchKernelGGL(k_qkv_sum_rope_rows, dim3((pairs + 255) / 256, n), dim3(256), 0, st, style, dim,
                     kv_dim, hd, ws, splits, ws_split, bq, bk, bv, q, ldq, k, ldk, v, ldv, pos0, n, sin_t,
                     cos_t);
  return launch_rc();
}

int kl::norm_planes_run(float* x, const float* w, int rows, int n, float eps, const float* ws,
                        int splits, size_t ws_split, void* planes, bool q8s, hipStream_t st) {
  if (!x || !w || !planes || rows <= 0 || n <= 0 || (splits > 0 && !ws) || (q8s && rows > 32))
    return KL_EINVAL;
  if (n % 32 || n > 8 * 256 * 4 || ws_split % 4 || !aligned16(x) || !aligned16(w) || !aligned16(planes))
    return KL_EUNSUPP;
  // Few rows (one workgroup each) summing several partials: the wide
  // reduction first (32 rows x 16 splits took 26 us in the row kernel).
  if (splits > 1 && rows < 128) {
    const int rr = partials_add_run(x, rows, n, ws, splits, st);
    if (rr != KL_OK) return rr;
    splits = 0;
  }
  // Few rows and no partials left (x is only read): the norm spread over up to
  // 8 workgroups per row, each storing a slice.
  const int slices = splits == 0 && rows < 128 ? std::max(1, std::min(8, 256 / rows)) : 1;
  const int r4 = (n / 4 + 255) / 256;
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(rows, slices), dim3(256), 0, st, x, w, n, eps, ws, splits, ws_split,
                       static_cast<__bf16*>(planes), q8s);
  };
  if (r4 <= 1) launch(k_norm_planes<1>);
  else if (r4 <= 2) launch(k_norm_planes<2>);
  else if (r4 <= 4) launch(k_norm_planes<4>);
  else launch(k_norm_planes<8>);
  return launch_rc();
}

int kl::swiglu_planes_run(const float* h1, const float* h3, int rows, int F, const float* ws, int splits,
                          size_t ws_split, size_t wsoff3, void* planes, bool q8s, hipStream_t st) {
  if (!planes || rows <= 0 || F <= 0 || (splits > 0 ? !ws : (!h1 || !h3)) || (q8s && rows > 32))
    return KL_EINVAL;
  if (F % 32 || ws_split % 4 || wsoff3 % 4 || !aligned16(planes)) return KL_EUNSUPP;
  const size_t work = static_cast<size_t>(rows) * (F / 4);
  const int grid = static_cast<int>(std::min<size_t>((work + 255) / 256, 8192));
  hipLaunchKernelGGL(k_swiglu_planes, dim3(grid), dim3(256), 0, st, h1, h3, rows, F, ws, splits,
                     ws_split, wsoff3, static_cast<__bf16*>(planes), q8s);
  return launch_rc();
}

int kl::partials_add_run(float* x, int rows, int n, const float* ws, int splits, hipStream_t st) {
  if (!x || !ws || rows <= 0 || n <= 0 || splits < 1) return KL_EINVAL;
  GemmArgs ra{};
  ra.M = rows;
  ra.accumulate = 1;
  ra.nseg = 1;
  ra.ws = const_cast<float*>(ws);
  ra.ws_split = static_cast<size_t>(rows) * n;
  ra.splits = splits;
  ra.seg[0].C = x;
  ra.seg[0].N = n;
  ra.seg[0].ldc = n;
  const int grid = static_cast<int>(std::min<size_t>((ra.ws_split + 255) / 256, 4096));
  hipLaunchKernelGGL(k_gemm_reduce, dim3(grid), dim3(256), 0, st, ra);
  return launch_rc();
}

int kl::x6_planes_flag_run(const void* planes, int rows, int K, unsigned* flag, hipStream_t st) {
  if (!planes || !flag || rows <= 0 || K <= 0) return KL_EINVAL;
  if (K % 32 || !aligned16(planes)) return KL_EUNSUPP;
  const size_t tiles = static_cast<size_t>((rows + 15) / 16) * (K / 32);
  const int grid = static_cast<int>(std::min<size_t>((tiles * 512 + 255) / 256, 4096));
  hipLaunchKernelGGL(k_x6_planes_nonzero, dim3(grid), dim3(256), 0, st,
                     static_cast<const unsigned*>(planes), rows, K, tiles, flag);
  return launch_rc();
}

int kl::split3_run(const float* x, int rows, int cols, int ldx, void* planes, hipStream_t st) {
  if (!x || !planes || rows <= 0 || cols <= 0 || ldx < cols) return KL_EINVAL;
  if (cols % 32 || ldx % 4 || !aligned16(x) || !aligned16(planes)) return KL_EUNSUPP;
  const size_t work = static_cast<size_t>(rows) * (cols / 8);
  const int grid = static_cast<int>(std::min<size_t>((work + 255) / 256, 8192));
  hipLaunchKernelGGL(k_split3, dim3(grid), dim3(256), 0, st, x, rows, cols, ldx,
                     static_cast<__bf16*>(planes));
  return launch_rc();
}

extern "C" {

size_t kl_split_bf16x3_bytes(int rows, int cols) {
  return rows > 0 && cols > 0 ? x6_plane_bytes(rows, cols) : 0;
}

int kl_split_bf16x3(const float* x, int rows, int cols, int ldx, void* planes, void* stream) {
  return split3_run(x, rows, cols, ldx, planes, as_stream(stream));
}

size_t kl_q8s_packed_bytes(int N, int K, int group_size) { return q8s_packed_bytes(N, K, group_size); }

int kl_q8s_pack(const int8_t* q, const float* scales, int N, int K, int group_size, void* packed,
                void* stream) {
  return q8s_pack_run(q, scales, N, K, group_size, packed, as_stream(stream));
}

int kl_gemm_q8s(const float* A, int M, int K, int lda, const void* packed, int N, int group_size,
                float* C, int ldc, const float* bias, int accumulate, void* workspace,
                size_t workspace_bytes, void* stream) {
  if (!C || N <= 0 || ldc < N || M <= 0 || M > 32) return KL_EINVAL;
  if (!workspace || workspace_bytes < q8s_aplane_bytes(K)) return KL_EWORKSPACE;
  hipStream_t st = as_stream(stream);
  int r = q8s_split_run(A, M, K, lda, workspace, st);
  if (r != KL_OK) return r;
  const size_t pb = (q8s_aplane_bytes(K) + 255) & ~size_t(255);
  float* ws = workspace_bytes > pb ? reinterpret_cast<float*>(static_cast<char*>(workspace) + pb) : nullptr;
  const GemmSeg sg{packed, C, bias, N, K, ldc, 0};
  return gemm_run_q8s(workspace, M, K, group_size, 1, &sg, accumulate, ws, ws ? workspace_bytes - pb : 0, st);
}

int kl_gemm_x6(const void* a_planes, const void* w_planes, float* C, int M, int N, int K, int ldc,
               const float* bias, int accumulate, void* workspace, size_t workspace_bytes,
               void* stream) {
  return kl_gemm_x6w(a_planes, w_planes, 3, C, M, N, K, ldc, bias, accumulate, workspace,
                     workspace_bytes, stream);
}

int kl_gemm_x6w(const void* a_planes, const void* w_planes, int w_planes_used, float* C, int M, int N,
                int K, int ldc, const float* bias, int accumulate, void* workspace,
                size_t workspace_bytes, void* stream) {
  if (!C || N <= 0 || ldc < N || (w_planes_used != 1 && w_planes_used != 3)) return KL_EINVAL;
  GemmX6Planes p{};
  p.A = a_planes;
  p.W[0] = w_planes;
  p.w_planes = w_planes_used;
  const GemmSeg sg{nullptr, C, bias, N, K, ldc, 0};
  return gemm_run_x6(p, M, K, 1, &sg, accumulate, static_cast<float*>(workspace), workspace_bytes,
                     as_stream(stream));
}

int kl_x6_weight_planes(const void* w_planes, int N, int K, int* planes_used, void* stream) {
  if (!planes_used) return KL_EINVAL;
  unsigned* flag = nullptr;
  if (hipMalloc(&flag, sizeof(unsigned)) != hipSuccess) return KL_ENOMEM;
  hipStream_t st = as_stream(stream);
  unsigned h = 0;
  int r = rc(hipMemsetAsync(flag, 0, sizeof(unsigned), st));
  if (r == KL_OK) r = x6_planes_flag_run(w_planes, N, K, flag, st);
  if (r == KL_OK) r = rc(hipMemcpyAsync(&h, flag, sizeof(unsigned), hipMemcpyDeviceToHost, st));
  if (r == KL_OK) r = rc(hipStreamSynchronize(st));
  (void)hipFree(flag);
  if (r == KL_OK) *planes_used = h ? 3 : 1;
  return r;
}

}  // extern "C"

namespace {
int device_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = kFaMaxWorkers;
  }
  return cus;
}

// Stream-K workgroups for a head size 64 / 128 prefill attention launch with
// a workspace: one per CU (at most kFaMaxWorkers, at most one per unit), or 0
// (one workgroup per segment) where equal ranges would not shorten the
// longest walk: the last row block's key blocks when the segments fit the
// CUs at once.
int attn_prefill_workers(int pos0, int n, int heads) {
  const FaGeom geo = fa_geom(pos0, n);
  const long long W = geo.wh * heads, segs = static_cast<long long>(geo.nqb) * heads;
  const long long G = std::min<long long>(std::min(device_cus(), kFaMaxWorkers), W);
  const long long per = (W + G - 1) / G;
  const long long plain = segs <= device_cus() ? geo.nk_last : (W + device_cus() - 1) / device_cus() + geo.nk_last;
  return per < plain ? static_cast<int>(G) : 0;
}

template <int HD>
int attn_prefill_launch(const float* q, int ldq, const float* kc, const float* vc, int kv_dim,
                        int kv_mul, int heads, float* out, int ldo, int pos0, int n, hipStream_t st,
                        float* part = nullptr) {
  // Head sizes 64 and 128 on the matrix cores (128: split bf16 products,
  // KL_PREFILL_ATTN=f32 keeps the fp32 products); 32 and 256 on the vector ALUs.
  constexpr bool kMfma = HD == 64 || HD == 128;
  const char* env = HD == 128 ? std::getenv("KL_PREFILL_ATTN") : nullptr;  // read per launch (tests switch it)
  const bool x6 = HD == 128 && !(env && std::strcmp(env, "f32") == 0);
  const void* fn = x6 ? reinterpret_cast<const void*>(&k_attn_prefill_x6)
                      : kMfma ? reinterpret_cast<const void*>(&k_attn_prefill_fa<kMfma ? HD : 64>)
                              : reinterpret_cast<const void*>(&k_attn_prefill<HD>);
  const size_t lds = x6 ? attn_prefill_x6_lds_bytes()
                        : kMfma ? attn_prefill_fa_lds_bytes(HD) : attn_prefill_lds_bytes(HD);
  static bool attr_set[2] = {false, false};  // per kernel of this head size
  if (!attr_set[x6]) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(lds));
    if (e != hipSuccess) return rc(e);
    attr_set[x6] = true;
  }
  const float scale = 1.f / std::sqrt(static_cast<float>(HD));
  const dim3 grid((n + kPrefillQB - 1) / kPrefillQB, heads);
  if constexpr (kMfma) {
    const int workers = part ? attn_prefill_workers(pos0, n, heads) : 0;
    const unsigned blocks = workers ? workers : grid.x * grid.y;
    if (x6)
      hipLaunchKernelGGL(k_attn_prefill_x6, dim3(blocks), dim3(512), lds, st, q, ldq, kc, vc,
                         kv_dim, kv_mul, out, ldo, pos0, n, scale, heads, workers ? part : nullptr);
    else
      hipLaunchKernelGGL(k_attn_prefill_fa<HD>, dim3(blocks), dim3(512), lds, st, q, ldq, kc, vc,
                         kv_dim, kv_mul, out, ldo, pos0, n, scale, heads, workers ? part : nullptr);
    if (workers) {
      const int r = launch_rc();
      if (r != KL_OK) return r;
      constexpr int kGroups = kPrefillQB / (256 / (HD / 4));  // merge workgroups per row block
      hipLaunchKernelGGL(k_attn_prefill_merge<HD>, dim3(grid.x * kGroups, heads), dim3(256), 0, st,
                         part, out, ldo, pos0, n, heads, workers);
    }
  } else {
    hipLaunchKernelGGL(k_attn_prefill<HD>, grid, dim3(256), lds, st, q, ldq, kc, vc, kv_dim, kv_mul,
                       out, ldo, pos0, n, scale);
  }
  return launch_rc();
}
}  // namespace

extern "C" {

int kl_attn_prefill(int pos0, int n_pos, int head_num, int kv_mul, int head_size, const float* q,
                    int ldq, const float* key_cache, const float* value_cache, int kv_dim,
                    float* out, int ldo, void* stream) {
  if (!q || !key_cache || !value_cache || !out || pos0 < 0 || n_pos <= 0 || n_pos > 65535 * 64 ||
      head_num <= 0 || kv_mul <= 0 || head_num % kv_mul != 0 ||
      kv_dim != head_num / kv_mul * head_size || ldq < head_num * head_size ||
      ldo < head_num * head_size)
    return KL_EINVAL;
  if (ldq % 4 || kv_dim % 4 || !aligned16(q) || !aligned16(key_cache) || !aligned16(value_cache))
    return KL_EUNSUPP;
  const hipStream_t st = as_stream(stream);
  switch (head_size) {
    case 32: return attn_prefill_launch<32>(q, ldq, key_cache, value_cache, kv_dim, kv_mul, head_num, out, ldo, pos0, n_pos, st);
    case 64: return attn_prefill_launch<64>(q, ldq, key_cache, value_cache, kv_dim, kv_mul, head_num, out, ldo, pos0, n_pos, st);
    case 128: return attn_prefill_launch<128>(q, ldq, key_cache, value_cache, kv_dim, kv_mul, head_num, out, ldo, pos0, n_pos, st);
    case 256: return attn_prefill_launch<256>(q, ldq, key_cache, value_cache, kv_dim, kv_mul, head_num, out, ldo, pos0, n_pos, st);
    default: return KL_EUNSUPP;
  }
}

int kl_attn_prefill_workspace_size(int n_pos, int head_num, int head_size, size_t* bytes) {
  if (!bytes || n_pos <= 0 || head_num <= 0 || head_size <= 0) return KL_EINVAL;
  *bytes = head_size == 64 || head_size == 128 ? attn_prefill_fa_ws_bytes(head_size) : 0;
  return KL_OK;
}

int kl_attn_prefill_ws(int pos0, int n_pos, int head_num, int kv_mul, int head_size, const float* q,
                       int ldq, const float* key_cache, const float* value_cache, int kv_dim,
                       float* out, int ldo, void* workspace, size_t workspace_bytes,
                       void* stream) {
  size_t need = 0;
  if (kl_attn_prefill_workspace_size(n_pos, head_num, head_size, &need) != KL_OK) return KL_EINVAL;
  if (need == 0 || pos0 < 0 || attn_prefill_workers(pos0, n_pos, head_num) == 0)
    return kl_attn_prefill(pos0, n_pos, head_num, kv_mul, head_size, q, ldq, key_cache,
                           value_cache, kv_dim, out, ldo, stream);
  if (!workspace || workspace_bytes < need) return KL_EWORKSPACE;
  if (!aligned16(workspace)) return KL_EUNSUPP;
  if (!q || !key_cache || !value_cache || !out || n_pos > 65535 * 64 || kv_mul <= 0 ||
      head_num % kv_mul != 0 || kv_dim != head_num / kv_mul * head_size ||
      ldq < head_num * head_size || ldo < head_num * head_size)
    return KL_EINVAL;
  if (ldq % 4 || ldo % 4 || kv_dim % 4 || !aligned16(q) || !aligned16(out) ||
      !aligned16(key_cache) || !aligned16(value_cache))
    return KL_EUNSUPP;
  const hipStream_t st = as_stream(stream);
  float* ws = static_cast<float*>(workspace);
  return head_size == 64
             ? attn_prefill_launch<64>(q, ldq, key_cache, value_cache, kv_dim, kv_mul, head_num, out,
                                       ldo, pos0, n_pos, st, ws)
             : attn_prefill_launch<128>(q, ldq, key_cache, value_cache, kv_dim, kv_mul, head_num,
                                        out, ldo, pos0, n_pos, st, ws);
}

int kl_swiglu(const float* a, const float* b, float* out, int n, void* stream) {
  if (!a || !b || !out || n <= 0) return KL_EINVAL;
  hipLaunchKernelGGL(k_swiglu, dim3(std::min((n + 255) / 256, 4096)), dim3(256), 0,
                     as_stream(stream), a, b, out, n);
  return launch_rc();
}

int kl_add(const float* a, const float* b, float* out, int n, void* stream) {
  if (!a || !b || !out || n <= 0) return KL_EINVAL;
  hipLaunchKernelGGL(k_add, dim3(std::min((n + 255) / 256, 4096)), dim3(256), 0, as_stream(stream),
                     a, b, out, n);
  return launch_rc();
}

int kl_scale(float scale, float* x, int n, void* stream) {
  if (!x || n <= 0) return KL_EINVAL;
  hipLaunchKernelGGL(k_scale, dim3(std::min((n + 255) / 256, 4096)), dim3(256), 0, as_stream(stream),
                     scale, x, n);
  return launch_rc();
}

int kl_softmax(float* x, int n, void* stream) {
  if (!x || n <= 0) return KL_EINVAL;
  hipLaunchKernelGGL(k_softmax_1, dim3(1), dim3(1024), 0, as_stream(stream), x, n);
  return launch_rc();
}

int kl_scale_sum(const float* value, const float* scale, float* out, int pos, int size, int stride,
                 void* stream) {
  if (!value || !scale || !out || pos < 0 || size <= 0 || stride < 0) return KL_EINVAL;
  if (pos > 0 && stride < size) return KL_EINVAL;  // rows may not overlap
  hipLaunchKernelGGL(k_scale_sum, dim3(std::min((size + 255) / 256, 4096)), dim3(256), 0,
                     as_stream(stream), value, scale, out, pos, size, stride);
  return launch_rc();
}

int kl_embedding(const int32_t* tokens, int n_tokens, const float* table, int vocab, int dim,
                 float* out, int32_t* bad_token_flag, void* stream) {
  if (!tokens || !table || !out || n_tokens <= 0 || vocab <= 0 || dim <= 0) return KL_EINVAL;
  hipLaunchKernelGGL(k_embedding, dim3(n_tokens), dim3(256), 0, as_stream(stream), tokens, table,
                     vocab, dim, out, bad_token_flag);
  return launch_rc();
}

int kl_hbm_probe(size_t bytes, int reps, float* read_gbps, float* copy_gbps) {
  if (!read_gbps || !copy_gbps || bytes < (size_t(1) << 20) || reps <= 0) return KL_EINVAL;
  bytes &= ~size_t(4095);
  constexpr int kThreads = 512;
  int dev = 0, cus = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err == hipSuccess) err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (err != hipSuccess) return rc(err);
  const int blocks = cus > 0 ? cus : 256;
  const size_t per = 2 * bytes / 16 / blocks;  // 16-byte elements per workgroup
  char* buf = nullptr;
  float* sink = nullptr;
  hipStream_t st = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  err = hipMalloc(&buf, 2 * bytes);
  if (err == hipSuccess) err = hipMalloc(&sink, sizeof(float) * blocks * kThreads);
  if (err == hipSuccess) err = hipStreamCreate(&st);
  if (err == hipSuccess) err = hipEventCreate(&e0);
  if (err == hipSuccess) err = hipEventCreate(&e1);
  if (err == hipSuccess) err = hipMemsetAsync(buf, 0, 2 * bytes, st);
  float ms_read = 0.f, ms_copy = 0.f;
  // Read probe over both halves (per * blocks * 16 bytes per repetition), one
  // warm-up run.
  for (int pass = 0; pass < 2 && err == hipSuccess; ++pass) {
    const int n = pass == 0 ? 1 : reps;
    err = hipEventRecord(e0, st);
    for (int r = 0; r < n && err == hipSuccess; ++r) {
      hipLaunchKernelGGL(k_read_probe, dim3(blocks), dim3(kThreads), 0, st,
                         reinterpret_cast<const kl::pf4*>(buf), per, sink);
      err = hipGetLastError();
    }
    if (err == hipSuccess) err = hipEventRecord(e1, st);
    if (err == hipSuccess) err = hipEventSynchronize(e1);
    if (err == hipSuccess) err = hipEventElapsedTime(&ms_read, e0, e1);
  }
  // Copy probe: the first half into the second (bytes read + bytes written).
  for (int pass = 0; pass < 2 && err == hipSuccess; ++pass) {
    const int n = pass == 0 ? 1 : reps;
    err = hipEventRecord(e0, st);
    for (int r = 0; r < n && err == hipSuccess; ++r)
      err = hipMemcpyAsync(buf + bytes, buf, bytes, hipMemcpyDeviceToDevice, st);
    if (err == hipSuccess) err = hipEventRecord(e1, st);
    if (err == hipSuccess) err = hipEventSynchronize(e1);
    if (err == hipSuccess) err = hipEventElapsedTime(&ms_copy, e0, e1);
  }
  if (err == hipSuccess) {
    *read_gbps = static_cast<float>(16.0 * per * blocks * reps / (ms_read * 1e-3) / 1e9);
    *copy_gbps = static_cast<float>(2.0 * bytes * reps / (ms_copy * 1e-3) / 1e9);
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (st) (void)hipStreamDestroy(st);
  if (sink) (void)hipFree(sink);
  if (buf) (void)hipFree(buf);
  return rc(err);
}

int kl_argmax_workspace_size(int n, size_t* bytes) {
  if (!bytes || n <= 0) return KL_EINVAL;
  const int g = argmax_blocks(n);
  *bytes = static_cast<size_t>(g) * (sizeof(float) + sizeof(int)) + 64;
  return KL_OK;
}

int kl_argmax(const float* x, int n, int32_t* out_index, void* workspace, size_t workspace_bytes,
              void* stream) {
  if (!x || !out_index || !workspace || n <= 0) return KL_EINVAL;
  size_t need = 0;
  kl_argmax_workspace_size(n, &need);
  if (workspace_bytes < need) return KL_EWORKSPACE;
  const int g = argmax_blocks(n);
  // Layout: counter (64 bytes reserved), values [g], indices [g].
  char* ws = static_cast<char*>(workspace);
  unsigned int* counter = reinterpret_cast<unsigned int*>(ws);
  float* pv = reinterpret_cast<float*>(ws + 64);
  int* pi = reinterpret_cast<int*>(ws + 64 + static_cast<size_t>(g) * sizeof(float));
  hipLaunchKernelGGL(k_argmax, dim3(g), dim3(256), 0, as_stream(stream), x, n, out_index, pv, pi,
                     counter);
  return launch_rc();
}

}  // extern "C"
