// Split-K decode attention over the contiguous KV cache (flash-decoding).
//
// Reference semantics (kernels/cpu/mha_kernel.cpp:5-61): for every query head
// h, kv head g = h / kv_mul, s_t = (q_h . K_t) / sqrt(hd) for t in [0, pos],
// softmax over t, out_h = sum_t p_t V_t.  Caches are [seq_len][kv_dim] per
// layer (the caller passes the layer base).
//
// Work split: one 256-thread workgroup per (kv head g, position chunk s).  A
// workgroup serves all kv_mul query heads of its kv head, so every K/V row it
// reads from HBM is used kv_mul times.  The chunk length adapts to the live
// context (chunk = max(min_chunk, ceil((pos+1)/G))); workgroups past the last
// chunk exit at once.  Each workgroup stores (o, m, l) for its chunk; the last
// workgroup of a kv head to finish (an atomic arrival counter, reset by that
// workgroup) merges the chunks with the usual rescaling
// O = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M).  A single chunk writes the
// output directly.
//
// With `transform` set, the kernel also applies what the reference runs
// between the K/V projections and attention (model/llama3.cpp:634-638,
// model/qwen3.cpp:485-500): the optional per-head RMSNorm of q and k, then
// RoPE at `pos`.  q is transformed in LDS; the workgroup owning position pos
// transforms K[pos] and writes it back to the cache, so later steps read the
// rotated key exactly as the reference's cache holds it.
#pragma once
#include <math.h>

#include "device.hpp"

namespace kl {

constexpr int kAttnMaxKvMul = 8;

struct AttnArgs {
  const float* q;          // [heads * HD]
  float* kcache;           // layer base, [seq_len][kv_dim]
  const float* vcache;     // layer base
  float* out;              // [heads * HD]
  float* part;             // [kv_heads][G][kv_mul][HD + 2]
  unsigned int* counters;  // [kv_heads], zero between launches
  const int* pos_ptr;      // device position (fused path) or nullptr
  int pos_val;
  int kv_dim, kv_mul, G, min_chunk, ch_max;
  int transform;           // 0: none, 1: RoPE, 2: per-head RMSNorm then RoPE
  int rope_style;          // 0 interleaved pairs, 1 rotate-half pairs
  const float* sin_t;      // [seq_len][HD]
  const float* cos_t;
  const float* qn;         // [HD] q norm weight (transform 2)
  const float* kn;         // [HD] k norm weight (transform 2)
  float qk_eps;
  float scale;             // 1 / sqrt(HD)
};

__host__ __device__ inline size_t attn_lds_floats(int hd, int kv_mul, int ch_max) {
  return static_cast<size_t>(kv_mul) * hd + static_cast<size_t>(kv_mul) * ch_max + hd +
         2 * kAttnMaxKvMul + static_cast<size_t>(256 / hd) * kv_mul * hd;
}

// Split plan shared by the op-level launcher and the fused engine: about 256
// workgroups in total (kv_heads * G), chunks of at least min_chunk positions.
struct MhaPlan {
  int G, min_chunk, ch_max;
  size_t part_floats, lds_bytes, ws_bytes;
};

inline MhaPlan mha_plan(int kv_heads, int kv_mul, int seq_len, int hd) {
  MhaPlan p;
  p.min_chunk = 16;
  int by_heads = 256 / (kv_heads > 0 ? kv_heads : 1);
  if (by_heads < 1) by_heads = 1;
  int by_len = (seq_len + p.min_chunk - 1) / p.min_chunk;
  if (by_len < 1) by_len = 1;
  p.G = by_heads < by_len ? by_heads : by_len;
  int ch = (seq_len + p.G - 1) / p.G;
  if (ch < p.min_chunk) ch = p.min_chunk;
  p.ch_max = (ch + 3) & ~3;
  p.part_floats = static_cast<size_t>(kv_heads) * p.G * kv_mul * (hd + 2);
  p.lds_bytes = attn_lds_floats(hd, kv_mul, p.ch_max) * sizeof(float);
  p.ws_bytes = ((p.part_floats * sizeof(float) + 255) & ~size_t(255)) +
               static_cast<size_t>(kv_heads) * sizeof(unsigned int);
  return p;
}

inline bool mha_shape_ok(int head_num, int kv_mul, int hd) {
  return head_num > 0 && kv_mul > 0 && head_num % kv_mul == 0 && kv_mul <= kAttnMaxKvMul &&
         (hd == 32 || hd == 64 || hd == 128 || hd == 256);
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_decode(AttnArgs a) {
  static_assert(HD % 4 == 0 && HD <= 256 && (256 % HD) == 0, "head size");
  extern __shared__ float lds[];
  constexpr int TPR = HD / 4;     // threads per key row
  constexpr int RPP = 256 / TPR;  // key rows per pass
  constexpr int NTG = 256 / HD;   // position groups in the PV product
  constexpr int HALF = HD / 2;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = blockIdx.x / a.G;
  const int s = blockIdx.x - g * a.G;
  const int kvm = a.kv_mul;
  const int pos = a.pos_ptr ? *a.pos_ptr : a.pos_val;
  const int n = pos + 1;
  int chunk = (n + a.G - 1) / a.G;
  if (chunk < a.min_chunk) chunk = a.min_chunk;
  const int nsplit = (n + chunk - 1) / chunk;
  if (s >= nsplit) return;  // uniform for the whole workgroup
  const int t0 = s * chunk;
  const int cnt = min(n, t0 + chunk) - t0;

  float* qs = lds;                    // [kvm][HD]
  float* sc = qs + kvm * HD;          // [kvm][ch_max]
  float* kp = sc + kvm * a.ch_max;    // [HD] transformed K[pos]
  float* ml = kp + HD;                // [2 * kAttnMaxKvMul] (m, l)
  float* red = ml + 2 * kAttnMaxKvMul;  // [NTG][kvm][HD]
  __shared__ int s_last;

  const float* qg = a.q + static_cast<size_t>(g) * kvm * HD;
  for (int i = tid; i < kvm * HD; i += 256) qs[i] = qg[i];
  __syncthreads();

  if (a.transform == 2) {
    // Per-head RMSNorm of q (kernels/cuda/rmsnorm_kernel.cu:8-60): one wave per head.
    for (int h = wave; h < kvm; h += kWavesPerBlock) {
      float ss = 0.f;
      for (int d = lane; d < HD; d += kWave) ss += qs[h * HD + d] * qs[h * HD + d];
      ss = wave_sum(ss);
      const float r = 1.f / sqrtf(ss / static_cast<float>(HD) + a.qk_eps);
      for (int d = lane; d < HD; d += kWave) qs[h * HD + d] = (r * qs[h * HD + d]) * a.qn[d];
    }
    __syncthreads();
  }
  if (a.transform >= 1) {
    const float* srow = a.sin_t + static_cast<size_t>(pos) * HD;
    const float* crow = a.cos_t + static_cast<size_t>(pos) * HD;
    for (int p = tid; p < kvm * HALF; p += 256) {
      const int h = p / HALF, j = p - h * HALF;
      const int i0 = a.rope_style ? h * HD + j : h * HD + 2 * j;
      const int i1 = a.rope_style ? i0 + HALF : i0 + 1;
      float v0 = qs[i0], v1 = qs[i1];
      rope_pair(v0, v1, crow[2 * j], srow[2 * j]);
      qs[i0] = v0;
      qs[i1] = v1;
    }
    // K[pos] of this kv head: done by wave 0 of the workgroup that owns pos,
    // in registers (each lane holds whole pairs), then written to the cache.
    if (wave == 0 && pos >= t0 && pos < t0 + cnt) {
      float* krow = a.kcache + static_cast<size_t>(pos) * a.kv_dim + static_cast<size_t>(g) * HD;
      constexpr int PPL = (HALF + kWave - 1) / kWave;  // pairs per lane
      float v0[PPL], v1[PPL];
      float ss = 0.f;
#pragma unroll
      for (int k = 0; k < PPL; ++k) {
        const int j = lane + k * kWave;
        if (j < HALF) {
          const int i0 = a.rope_style ? j : 2 * j;
          const int i1 = a.rope_style ? j + HALF : 2 * j + 1;
          v0[k] = krow[i0];
          v1[k] = krow[i1];
          ss += v0[k] * v0[k] + v1[k] * v1[k];
        }
      }
      float r = 1.f;
      if (a.transform == 2) {
        ss = wave_sum(ss);
        r = 1.f / sqrtf(ss / static_cast<float>(HD) + a.qk_eps);
      }
#pragma unroll
      for (int k = 0; k < PPL; ++k) {
        const int j = lane + k * kWave;
        if (j < HALF) {
          const int i0 = a.rope_style ? j : 2 * j;
          const int i1 = a.rope_style ? j + HALF : 2 * j + 1;
          float x0 = v0[k], x1 = v1[k];
          if (a.transform == 2) {
            x0 = (r * x0) * a.kn[i0];
            x1 = (r * x1) * a.kn[i1];
          }
          rope_pair(x0, x1, crow[2 * j], srow[2 * j]);
          krow[i0] = x0;
          krow[i1] = x1;
          kp[i0] = x0;
          kp[i1] = x1;
        }
      }
    }
    __syncthreads();
  }

  // Scores: TPR lanes per key row, every row used for all kvm query heads.
  {
    const int sub = tid % TPR;
    const f4* q4 = reinterpret_cast<const f4*>(qs);
    const int passes = (cnt + RPP - 1) / RPP;
    for (int ps = 0; ps < passes; ++ps) {
      const int tt = ps * RPP + tid / TPR;
      const bool valid = tt < cnt;
      const int t = t0 + (valid ? tt : 0);
      const float* krow = (a.transform >= 1 && t == pos)
                              ? kp
                              : a.kcache + static_cast<size_t>(t) * a.kv_dim +
                                    static_cast<size_t>(g) * HD;
      const f4 k4 = reinterpret_cast<const f4*>(krow)[sub];
#pragma unroll
      for (int h = 0; h < kAttnMaxKvMul; ++h) {
        if (h < kvm) {
          float d = hsum(k4 * q4[h * TPR + sub]);
          d = group_sum(d, TPR);
          if (valid && sub == 0) sc[h * a.ch_max + tt] = d * a.scale;
        }
      }
    }
  }
  __syncthreads();

  // Chunk-local softmax statistics, one wave per head.
  for (int h = wave; h < kvm; h += kWavesPerBlock) {
    float* sh = sc + h * a.ch_max;
    float m = -INFINITY;
    for (int tt = lane; tt < cnt; tt += kWave) m = fmaxf(m, sh[tt]);
    m = wave_max(m);
    float l = 0.f;
    for (int tt = lane; tt < cnt; tt += kWave) {
      const float p = expf(sh[tt] - m);
      sh[tt] = p;
      l += p;
    }
    l = wave_sum(l);
    if (lane == 0) {
      ml[2 * h] = m;
      ml[2 * h + 1] = l;
    }
  }
  __syncthreads();

  // o_h[d] = sum_t p_h[t] V_t[d]; NTG position groups, reduced through LDS.
  const int d = tid % HD;
  const int tg = tid / HD;
  float o[kAttnMaxKvMul];
#pragma unroll
  for (int h = 0; h < kAttnMaxKvMul; ++h) o[h] = 0.f;
  for (int tt = tg; tt < cnt; tt += NTG) {
    const float v =
        a.vcache[static_cast<size_t>(t0 + tt) * a.kv_dim + static_cast<size_t>(g) * HD + d];
#pragma unroll
    for (int h = 0; h < kAttnMaxKvMul; ++h)
      if (h < kvm) o[h] += sc[h * a.ch_max + tt] * v;
  }
  if constexpr (NTG > 1) {
#pragma unroll
    for (int h = 0; h < kAttnMaxKvMul; ++h)
      if (h < kvm) red[(tg * kvm + h) * HD + d] = o[h];
    __syncthreads();
    if (tg == 0) {
#pragma unroll
      for (int h = 0; h < kAttnMaxKvMul; ++h) {
        if (h < kvm) {
          float t = o[h];
          for (int k = 1; k < NTG; ++k) t += red[(k * kvm + h) * HD + d];
          o[h] = t;
        }
      }
    }
  }

  float* outg = a.out + static_cast<size_t>(g) * kvm * HD;
  if (nsplit == 1) {
    if (tg == 0) {
#pragma unroll
      for (int h = 0; h < kAttnMaxKvMul; ++h)
        if (h < kvm) outg[h * HD + d] = o[h] / ml[2 * h + 1];
    }
    return;
  }

  float* pg = a.part + static_cast<size_t>(g) * a.G * kvm * (HD + 2);
  if (tg == 0) {
    float* ps = pg + static_cast<size_t>(s) * kvm * (HD + 2);
#pragma unroll
    for (int h = 0; h < kAttnMaxKvMul; ++h) {
      if (h < kvm) {
        ps[h * (HD + 2) + d] = o[h];
        if (d == 0) {
          ps[h * (HD + 2) + HD] = ml[2 * h];
          ps[h * (HD + 2) + HD + 1] = ml[2 * h + 1];
        }
      }
    }
    __threadfence();
  }
  __syncthreads();
  if (tid == 0) {
    const unsigned int prev = atomicAdd(a.counters + g, 1u);
    s_last = (prev == static_cast<unsigned int>(nsplit - 1)) ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  for (int idx = tid; idx < kvm * HD; idx += 256) {
    const int h = idx / HD, dd = idx - h * HD;
    float M = -INFINITY;
    for (int k = 0; k < nsplit; ++k)
      M = fmaxf(M, pg[(static_cast<size_t>(k) * kvm + h) * (HD + 2) + HD]);
    float L = 0.f, O = 0.f;
    for (int k = 0; k < nsplit; ++k) {
      const float* pk = pg + (static_cast<size_t>(k) * kvm + h) * (HD + 2);
      const float w = expf(pk[HD] - M);
      L += pk[HD + 1] * w;
      O += pk[dd] * w;
    }
    outg[h * HD + dd] = O / L;
  }
  if (tid == 0) a.counters[g] = 0u;
}

}  // namespace kl
