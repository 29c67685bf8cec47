// Causal attention of a batch of prompt positions for the batched prefill:
// the semantics of kernels/cpu/mha_kernel.cpp:5-61 (per head h, kv head
// h / kv_mul: softmax_t((q_h . K_t) / sqrt(hd)) . V_t over t <= position) for
// query positions pos0 .. pos0 + n - 1 at once, reading K and V rows 0 ..
// pos0 + n - 1 of one layer's caches ([seq_len][kv_dim]).
//
// One workgroup (256 threads) owns 64 query rows of one head and walks the
// key positions in blocks of 64 through LDS with an online softmax: thread
// (rg, cg) = (tid / 16, tid % 16) scores rows 4 rg .. 4 rg + 3 against keys
// 4 cg .. 4 cg + 3 of the block, the 16 threads of a row group combine the
// row maxima and sums with lane shuffles, and the same thread accumulates
// output columns cg * HD / 16 .. of its 4 rows.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>

namespace kl {

typedef float pf4 __attribute__((ext_vector_type(4)));

constexpr int kPrefillQB = 64;  // query rows per workgroup
constexpr int kPrefillKB = 64;  // key positions per block

__host__ __device__ constexpr size_t attn_prefill_lds_bytes(int hd) {
  return (static_cast<size_t>(kPrefillQB + 2 * kPrefillKB) * (hd + 4) +
          static_cast<size_t>(kPrefillQB) * (kPrefillKB + 4)) * sizeof(float);
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_prefill(const float* __restrict__ q, int ldq,
                                                      const float* __restrict__ kc,
                                                      const float* __restrict__ vc, int kv_dim,
                                                      int kv_mul, float* __restrict__ out, int ldo,
                                                      int pos0, int n, float scale) {
  constexpr int QB = kPrefillQB, KB = kPrefillKB, LD = HD + 4, LP = KB + 4, DPT = HD / 16;
  extern __shared__ __align__(16) float sm[];
  float* Qs = sm;
  float* Ks = Qs + QB * LD;
  float* Vs = Ks + KB * LD;
  float* Ps = Vs + KB * LD;
  const int h = blockIdx.y, g = h / kv_mul;
  const int p0 = blockIdx.x * QB;
  const int tid = threadIdx.x, rg = tid >> 4, cg = tid & 15;

  for (int i = tid; i < QB * HD / 4; i += 256) {
    const int r = i / (HD / 4), c = 4 * (i % (HD / 4));
    const int p = p0 + r;
    const pf4 v = p < n ? *reinterpret_cast<const pf4*>(q + static_cast<size_t>(p) * ldq + h * HD + c)
                        : pf4{0.f, 0.f, 0.f, 0.f};
    *reinterpret_cast<pf4*>(Qs + r * LD + c) = v;
  }
  float m[4], l[4], o[4][DPT];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    m[a] = -INFINITY;
    l[a] = 0.f;
#pragma unroll
    for (int c = 0; c < DPT; ++c) o[a][c] = 0.f;
  }
  const int rows = n - p0 < QB ? n - p0 : QB;
  const int last = pos0 + p0 + rows - 1;  // last key any row of the block attends
  for (int j0 = 0; j0 <= last; j0 += KB) {
    __syncthreads();  // the previous block's K, V and P are consumed
    for (int i = tid; i < KB * HD / 4; i += 256) {
      const int r = i / (HD / 4), c = 4 * (i % (HD / 4));
      const int j = j0 + r;
      const size_t off = static_cast<size_t>(j <= last ? j : 0) * kv_dim + g * HD + c;
      const pf4 kv = *reinterpret_cast<const pf4*>(kc + off);
      const pf4 vv = *reinterpret_cast<const pf4*>(vc + off);
      *reinterpret_cast<pf4*>(Ks + r * LD + c) = j <= last ? kv : pf4{0.f, 0.f, 0.f, 0.f};
      *reinterpret_cast<pf4*>(Vs + r * LD + c) = j <= last ? vv : pf4{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();
    float s[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) s[a][b] = 0.f;
    for (int d = 0; d < HD; d += 4) {
      pf4 qv[4], kv[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) qv[a] = *reinterpret_cast<const pf4*>(Qs + (4 * rg + a) * LD + d);
#pragma unroll
      for (int b = 0; b < 4; ++b) kv[b] = *reinterpret_cast<const pf4*>(Ks + (4 * cg + b) * LD + d);
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
          s[a][b] += qv[a].x * kv[b].x + qv[a].y * kv[b].y + qv[a].z * kv[b].z + qv[a].w * kv[b].w;
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int qpos = pos0 + p0 + 4 * rg + a;
      float mx = -INFINITY;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int kpos = j0 + 4 * cg + b;
        s[a][b] = kpos <= qpos ? s[a][b] * scale : -INFINITY;
        mx = fmaxf(mx, s[a][b]);
      }
#pragma unroll
      for (int w = 1; w < 16; w <<= 1) mx = fmaxf(mx, __shfl_xor(mx, w, 16));
      const float mn = fmaxf(m[a], mx);
      // Key 0 is in the first block for every row, so mn is finite from then on.
      const float alpha = m[a] == -INFINITY ? 0.f : expf(m[a] - mn);
      float rs = 0.f;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const float pv = s[a][b] == -INFINITY ? 0.f : expf(s[a][b] - mn);
        Ps[(4 * rg + a) * LP + 4 * cg + b] = pv;
        rs += pv;
      }
#pragma unroll
      for (int w = 1; w < 16; w <<= 1) rs += __shfl_xor(rs, w, 16);
      l[a] = l[a] * alpha + rs;
      m[a] = mn;
#pragma unroll
      for (int c = 0; c < DPT; ++c) o[a][c] *= alpha;
    }
    __syncthreads();
    const int jn = last - j0 + 1 < KB ? last - j0 + 1 : KB;
    for (int j = 0; j < jn; ++j) {
      float pj[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) pj[a] = Ps[(4 * rg + a) * LP + j];
      const float* vr = Vs + j * LD + cg * DPT;
#pragma unroll
      for (int c = 0; c < DPT; ++c) {
        const float v = vr[c];
#pragma unroll
        for (int a = 0; a < 4; ++a) o[a][c] += pj[a] * v;
      }
    }
  }
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int p = p0 + 4 * rg + a;
    if (p < n) {
      float* op = out + static_cast<size_t>(p) * ldo + h * HD + cg * DPT;
#pragma unroll
      for (int c = 0; c < DPT; ++c) op[c] = o[a][c] / l[a];
    }
  }
}

}  // namespace kl
