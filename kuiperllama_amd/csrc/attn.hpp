// Split-K decode attention over the contiguous KV cache (flash-decoding).
//
// Reference semantics (kernels/cpu/mha_kernel.cpp:5-61): for every query head
// h, kv head g = h / kv_mul, s_t = (q_h . K_t) / sqrt(hd) for t in [0, pos],
// softmax over t, out_h = sum_t p_t V_t.  Caches are [seq_len][kv_dim] per
// layer (the caller passes the layer base).
//
// Work split: one 256-thread workgroup per (kv head g, span of cpw chunks of
// PT positions); the grid covers the whole cache and workgroups past the live
// context exit at once.  A workgroup serves all kv_mul query heads of its kv
// head, so each K/V row read from HBM is used kv_mul times.  Every K and V
// load of a chunk is issued at once into registers (HD/4 lanes per row,
// PT/(1024/HD) rows per lane), so a chunk costs one memory round trip; q
// staging, q/k normalisation and RoPE overlap with the first.  The chunks of
// a span are folded with a running maximum (o, m, l).  Each workgroup stores
// (o, m, l) of its span; the spans of a kv head are merged with
// O = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M), either by the last
// workgroup to finish (atomic arrival counter, reset by that workgroup; the
// fused engine) or by k_attn_merge launched after it (no counter, so the
// workspace needs no initialisation; the op-level entry point).  A single
// span writes the output directly.
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
  unsigned int* counters;  // [kv_heads], zero between launches; nullptr: k_attn_merge merges
  const int* pos_ptr;      // device position (fused path) or nullptr
  int pos_val;
  int kv_dim, kv_mul, G;   // G: span slots per kv head = ceil(ceil(seq_len / PT) / cpw)
  int cpw;                 // chunks of PT positions per workgroup (span)
  int transform;           // 0: none, 1: RoPE, 2: per-head RMSNorm then RoPE
  int rope_style;          // 0 interleaved pairs, 1 rotate-half pairs
  const float* sin_t;      // [seq_len][HD]
  const float* cos_t;
  const float* qn;         // [HD] q norm weight (transform 2)
  const float* kn;         // [HD] k norm weight (transform 2)
  float qk_eps;
  float scale;             // 1 / sqrt(HD)
};

// Positions per workgroup for a head size (8 K and 8 V chunks per lane at
// most: 64 VGPRs of prefetched cache).
__host__ __device__ constexpr int attn_chunk(int hd) { return hd >= 256 ? 32 : 64; }

__host__ __device__ inline size_t attn_lds_floats(int hd, int kv_mul) {
  const int pt = attn_chunk(hd);
  const int rpp = 256 / (hd / 4);
  return static_cast<size_t>(kv_mul) * hd      // q
         + static_cast<size_t>(kv_mul) * pt    // scores
         + hd                                  // transformed K[pos]
         + 4 * kAttnMaxKvMul                   // chunk (m, l), span (m, l)
         + static_cast<size_t>(rpp) * kv_mul * hd;  // PV reduction
}

// Split plan shared by the op-level launcher and the fused engine.
struct MhaPlan {
  int G;    // spans (workgroups) per kv head
  int cpw;  // chunks per span
  size_t part_floats, lds_bytes;
  size_t ws_bytes;  // part + arrival counters (the fused engine's layout)
};

inline MhaPlan mha_plan(int kv_heads, int kv_mul, int seq_len, int hd, int cpw = 1) {
  MhaPlan p;
  const int pt = attn_chunk(hd);
  const int chunks = (seq_len + pt - 1) / pt;
  p.cpw = cpw;
  p.G = (chunks + cpw - 1) / cpw;
  p.part_floats = static_cast<size_t>(kv_heads) * p.G * kv_mul * (hd + 2);
  p.lds_bytes = attn_lds_floats(hd, kv_mul) * sizeof(float);
  p.ws_bytes = ((p.part_floats * sizeof(float) + 255) & ~size_t(255)) +
               static_cast<size_t>(kv_heads) * sizeof(unsigned int);
  return p;
}

// The op-level plan: the fewest chunks per span whose partials fit the
// reference's score buffer, head_num x seq_len floats (llama3.cpp:485-487).
// A plan with one span per kv head needs no workspace at all.
inline MhaPlan mha_plan_fit(int head_num, int kv_mul, int seq_len, int hd, size_t* ws_bytes) {
  const int kv_heads = head_num / kv_mul;
  const size_t budget = static_cast<size_t>(head_num) * seq_len * sizeof(float);
  const int chunks = (seq_len + attn_chunk(hd) - 1) / attn_chunk(hd);
  for (int cpw = 1;; ++cpw) {
    MhaPlan p = mha_plan(kv_heads, kv_mul, seq_len, hd, cpw);
    const size_t need = p.G > 1 ? p.part_floats * sizeof(float) : 0;
    if (need <= budget || cpw >= chunks) {
      *ws_bytes = need;
      return p;
    }
  }
}

inline bool mha_shape_ok(int head_num, int kv_mul, int hd) {
  return head_num > 0 && kv_mul > 0 && head_num % kv_mul == 0 && kv_mul <= kAttnMaxKvMul &&
         (hd == 32 || hd == 64 || hd == 128 || hd == 256);
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_decode(AttnArgs a) {
  static_assert(HD % 4 == 0 && HD <= 256 && (256 % HD) == 0, "head size");
  constexpr int PT = attn_chunk(HD);  // positions per chunk
  constexpr int TPR = HD / 4;         // lanes per key row (one f4 each)
  constexpr int RPP = 256 / TPR;      // rows per pass
  constexpr int NP = PT / RPP;        // passes: rows per lane
  constexpr int HALF = HD / 2;
  constexpr int OPT = (kAttnMaxKvMul * HD + 255) / 256;  // outputs per thread, at most
  static_assert(NP >= 1 && NP * RPP == PT, "chunk geometry");
  extern __shared__ float lds[];
  __shared__ int s_last;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int sub = tid % TPR;  // which f4 of the row
  const int rr = tid / TPR;   // row within a pass
  const int g = blockIdx.x / a.G;
  const int s = blockIdx.x - g * a.G;
  const int kvm = a.kv_mul;
  const int pos = a.pos_ptr ? *a.pos_ptr : a.pos_val;
  const int n = pos + 1;
  const int span = PT * a.cpw;
  const int nsplit = (n + span - 1) / span;
  if (s >= nsplit) return;  // uniform for the whole workgroup
  const int w0 = s * span;
  const int wcnt = min(n - w0, span);
  const int nsub = (wcnt + PT - 1) / PT;
  const bool own_pos = pos >= w0 && pos < w0 + wcnt;
  const size_t col = static_cast<size_t>(g) * HD + 4 * sub;

  // 1. The first chunk's K and V rows, straight into registers.
  f4 kr[NP], vr[NP];
  auto load_chunk = [&](int t0, int cnt) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int tt = p * RPP + rr;
      const size_t off = static_cast<size_t>(t0 + (tt < cnt ? tt : 0)) * a.kv_dim + col;
      kr[p] = *reinterpret_cast<const f4*>(a.kcache + off);
      vr[p] = *reinterpret_cast<const f4*>(a.vcache + off);
    }
  };
  load_chunk(w0, min(wcnt, PT));

  float* qs = lds;                 // [kvm][HD]
  float* sc = qs + kvm * HD;       // [kvm][PT]
  float* kp = sc + kvm * PT;       // [HD]
  float* ml = kp + HD;             // [2 * kAttnMaxKvMul] chunk (m, l)
  float* run = ml + 2 * kAttnMaxKvMul;  // [2 * kAttnMaxKvMul] span (m, l)
  float* red = run + 2 * kAttnMaxKvMul;  // [RPP][kvm][HD]

  // 2. q of the group's heads (and its transforms), K[pos] transform.
  const float* qg = a.q + static_cast<size_t>(g) * kvm * HD;
  for (int i = tid; i < kvm * HD; i += 256) qs[i] = qg[i];
  if (tid < kvm) {
    run[2 * tid] = -INFINITY;
    run[2 * tid + 1] = 0.f;
  }
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
    // K[pos] of this kv head: wave 0 of the workgroup owning pos, in registers
    // (each lane holds whole pairs), then written back to the cache and kept
    // in LDS for the chunk that holds pos.
    if (wave == 0 && own_pos) {
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
  }
  __syncthreads();

  // Span accumulators: thread tid owns outputs idx = tid + 256 * j.
  float ro[OPT];
#pragma unroll
  for (int j = 0; j < OPT; ++j) ro[j] = 0.f;

  for (int c = 0; c < nsub; ++c) {
    const int t0 = w0 + c * PT;
    const int cnt = min(w0 + wcnt - t0, PT);
    if (c > 0) load_chunk(t0, cnt);
    if (a.transform >= 1 && pos >= t0 && pos < t0 + cnt) {
      // The lane that loaded K[pos] (raw) takes the transformed row.
#pragma unroll
      for (int p = 0; p < NP; ++p)
        if (t0 + p * RPP + rr == pos) kr[p] = reinterpret_cast<const f4*>(kp)[sub];
    }

    // 3. Scores: TPR lanes per key row, each row used for all kvm query heads.
    {
      const f4* q4 = reinterpret_cast<const f4*>(qs);
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int tt = p * RPP + rr;
#pragma unroll
        for (int h = 0; h < kAttnMaxKvMul; ++h) {
          if (h < kvm) {
            float d = hsum(kr[p] * q4[h * TPR + sub]);
            d = group_sum(d, TPR);
            if (sub == 0 && tt < cnt) sc[h * PT + tt] = d * a.scale;
          }
        }
      }
    }
    __syncthreads();

    // 4. Chunk-local softmax statistics, one wave per head.
    for (int h = wave; h < kvm; h += kWavesPerBlock) {
      float* sh = sc + h * PT;
      float m = -INFINITY;
      for (int tt = lane; tt < cnt; tt += kWave) m = fmaxf(m, sh[tt]);
      m = wave_max(m);
      float l = 0.f;
      for (int tt = lane; tt < cnt; tt += kWave) {
        const float e = expf(sh[tt] - m);
        sh[tt] = e;
        l += e;
      }
      l = wave_sum(l);
      if (lane == 0) {
        ml[2 * h] = m;
        ml[2 * h + 1] = l;
      }
    }
    __syncthreads();

    // 5. o_h = sum_t p_h[t] V_t: per-lane partials over its rows, then summed
    //    over the RPP row slots through LDS and folded into the span.
#pragma unroll
    for (int h = 0; h < kAttnMaxKvMul; ++h) {
      if (h < kvm) {
        f4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const int tt = p * RPP + rr;
          if (tt < cnt) o += sc[h * PT + tt] * vr[p];
        }
        reinterpret_cast<f4*>(red + (static_cast<size_t>(rr) * kvm + h) * HD)[sub] = o;
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < OPT; ++j) {
      const int idx = tid + 256 * j;
      if (idx < kvm * HD) {
        const int h = idx / HD, d = idx - h * HD;
        float o = 0.f;
        for (int k = 0; k < RPP; ++k) o += red[(static_cast<size_t>(k) * kvm + h) * HD + d];
        const float mo = run[2 * h], mc = ml[2 * h];
        const float mn = fmaxf(mo, mc);
        ro[j] = ro[j] * expf(mo - mn) + o * expf(mc - mn);
      }
    }
    __syncthreads();
    if (tid < kvm) {
      const float mo = run[2 * tid], mc = ml[2 * tid];
      const float mn = fmaxf(mo, mc);
      run[2 * tid + 1] = run[2 * tid + 1] * expf(mo - mn) + ml[2 * tid + 1] * expf(mc - mn);
      run[2 * tid] = mn;
    }
    __syncthreads();
  }

  float* outg = a.out + static_cast<size_t>(g) * kvm * HD;
  float* pg = a.part + static_cast<size_t>(g) * a.G * kvm * (HD + 2);
#pragma unroll
  for (int j = 0; j < OPT; ++j) {
    const int idx = tid + 256 * j;
    if (idx < kvm * HD) {
      const int h = idx / HD, d = idx - h * HD;
      if (nsplit == 1) {
        outg[h * HD + d] = ro[j] / run[2 * h + 1];
      } else {
        float* ps = pg + (static_cast<size_t>(s) * kvm + h) * (HD + 2);
        store_coherent(ps + d, ro[j]);
        if (d == 0) {
          store_coherent(ps + HD, run[2 * h]);
          store_coherent(ps + HD + 1, run[2 * h + 1]);
        }
      }
    }
  }
  if (nsplit == 1 || !a.counters) return;

  wait_mem();
  __syncthreads();
  if (tid == 0) {
    const unsigned int prev = arrive(a.counters + g);
    s_last = (prev == static_cast<unsigned int>(nsplit - 1)) ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;
  // 6. Merge the spans of this kv head.  The (m, l) pairs go through LDS
  //    once; the o rows are read in one pass.
  float* mls = red;  // reuse: [nsplit][kvm][2]
  for (int i = tid; i < nsplit * kvm; i += 256) {
    const float* pk = pg + static_cast<size_t>(i) * (HD + 2);
    mls[2 * i] = load_coherent(pk + HD);
    mls[2 * i + 1] = load_coherent(pk + HD + 1);
  }
  __syncthreads();
  for (int idx = tid; idx < kvm * HD; idx += 256) {
    const int h = idx / HD, d = idx - h * HD;
    float M = -INFINITY;
    for (int k = 0; k < nsplit; ++k) M = fmaxf(M, mls[2 * (k * kvm + h)]);
    float L = 0.f, O = 0.f;
    for (int k = 0; k < nsplit; ++k) {
      const float w = expf(mls[2 * (k * kvm + h)] - M);
      L += mls[2 * (k * kvm + h) + 1] * w;
      O += load_coherent(pg + (static_cast<size_t>(k) * kvm + h) * (HD + 2) + d) * w;
    }
    outg[h * HD + d] = O / L;
  }
  if (tid == 0) a.counters[g] = 0u;
}

// The merge of step 6 as its own launch (grid: one workgroup per kv head),
// after k_attn_decode ran without arrival counters.  Same order of operations
// as the in-kernel merge.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_merge(AttnArgs a) {
  extern __shared__ float lds[];
  constexpr int PT = attn_chunk(HD);
  const int tid = threadIdx.x;
  const int g = blockIdx.x;
  const int kvm = a.kv_mul;
  const int pos = a.pos_ptr ? *a.pos_ptr : a.pos_val;
  const int nsplit = (pos + PT * a.cpw) / (PT * a.cpw);
  if (nsplit <= 1) return;
  const float* pg = a.part + static_cast<size_t>(g) * a.G * kvm * (HD + 2);
  float* outg = a.out + static_cast<size_t>(g) * kvm * HD;
  float* mls = lds;  // [nsplit][kvm][2]
  for (int i = tid; i < nsplit * kvm; i += 256) {
    const float* pk = pg + static_cast<size_t>(i) * (HD + 2);
    mls[2 * i] = pk[HD];
    mls[2 * i + 1] = pk[HD + 1];
  }
  __syncthreads();
  for (int idx = tid; idx < kvm * HD; idx += 256) {
    const int h = idx / HD, d = idx - h * HD;
    float M = -INFINITY;
    for (int k = 0; k < nsplit; ++k) M = fmaxf(M, mls[2 * (k * kvm + h)]);
    float L = 0.f, O = 0.f;
    for (int k = 0; k < nsplit; ++k) {
      const float w = expf(mls[2 * (k * kvm + h)] - M);
      L += mls[2 * (k * kvm + h) + 1] * w;
      O += pg[(static_cast<size_t>(k) * kvm + h) * (HD + 2) + d] * w;
    }
    outg[h * HD + d] = O / L;
  }
}

}  // namespace kl
