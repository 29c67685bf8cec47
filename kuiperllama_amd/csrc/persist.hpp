// Persistent decode step: one cooperative launch runs a whole token of the
// reference forward (model/llama3.cpp:146-166, :599-744; qwen2.cpp:205-225;
// qwen3.cpp:147-167) on every CU at once.
//
// Phases of one token, separated by grid barriers:
//   per layer:  QKV GEMV -> attention -> WO GEMV -> W1/W3 GEMV -> W2 GEMV
//   then:       classifier GEMV + argmax (sampled positions only)
//
// Why persistent: a decode step of Llama-3.2-1B streams 4.9 GB of weights in
// 81 GEMV-shaped pieces, most of them 17-67 MB.  As separate kernels each pays
// a launch, a ramp-up and a drain, and the small ones never reach full HBM
// bandwidth.  Here every wave keeps streaming weights across phase
// boundaries: weights do not depend on activations, so each wave issues the
// loads of its first batch of the NEXT GEMV phase before it waits at the
// barrier (and across the attention phase), and HBM stays busy while the
// barrier, the activation hand-off and the attention run.
//
// GEMV phases.  The split dimension (output rows) is cut into one contiguous
// range per workgroup.  Inside the workgroup, KS waves share a row (split-K)
// and RW = 8 / KS row groups take rows round robin; the host planner picks KS
// per phase.  A wave's work is a list of items = (local row, 1 KiB column
// chunk): 64 lanes x 16 bytes (4 fp32 or 16 int8 weights per lane).  Items
// are streamed through two register buffers of NB items each (double
// buffering); a wave's partial sum for a row is reduced across the wave and
// stored to LDS slot [row][k-slice], so the sum order is fixed (results are
// bitwise reproducible).  The epilogue combines the KS slices per row.
//
// Hand-off between workgroups.  Activations written by one workgroup and read
// by another (q, K/V rows, attention output, residual stream, FFN hidden
// vector) are stored with agent-coherent (sc1) stores and read with coherent
// loads, so no L2 of the eight XCDs can serve a stale copy; each thread drains
// its stores before its workgroup arrives at the barrier.  Weights, norms and
// tables are read-only during the launch and use ordinary (nontemporal) loads.
//
// Barrier.  A monotonically increasing arrival counter; barrier k of a launch
// waits until the counter reaches base + (k+1) * gridDim.x, where base is
// carried from launch to launch in device memory.  The wait is bounded: after
// kSpinLimit polls the workgroup records an error and every later barrier of
// the launch returns at once, so every wave always reaches the end of the
// kernel; the host reports the error.
#pragma once
#include <math.h>

#include "attn.hpp"
#include "device.hpp"

namespace kl {

constexpr int kPThreads = 512;
constexpr int kPWaves = kPThreads / kWave;
constexpr int kSpinLimit = 1 << 22;

// Error codes written to PArgs::err by the device.
constexpr int kDevErrBarrier = 1;  // a barrier wait exceeded kSpinLimit polls
constexpr int kDevErrPos = 2;      // position outside [0, seq_len)
constexpr int kDevErrToken = 3;    // the sampler found no finite maximum

enum : int { kEpiQkv = 0, kEpiResid = 1, kEpiSwiglu = 2, kEpiCls = 3 };

// One GEMV phase (host-built, read-only in device memory).
struct PGemv {
  const void* w[3];       // sub-matrices, row-major [rows x cols]; fp32 or int8
  const float* sc[3];     // int8: one fp32 scale per 2^gshift consecutive elements
  int rows[3];
  int nsub;               // 1..3
  int paired;             // 0: sub-matrix rows are concatenated and split; 1: every
                          //    workgroup takes the same row range of each sub-matrix
  int cols;
  int cn;                 // 1 KiB chunks per row (last one may be partial)
  int cn16;               // 16-byte lane units per row
  int gshift;             // int8 group size = 1 << gshift
  int rpw;                // split-dimension rows per workgroup
  int ks, rw;             // waves per row (split-K), row groups; ks * rw == kPWaves
  int nck;                // chunks per (row, k-slice) = ceil(cn / ks)
  int epi;                // kEpi*
  const float* in;        // input vector; nullptr: embedding row of the step's token
  const float* norm;      // RMSNorm weight applied to the input, or nullptr
  float* out[3];          // qkv: q, K cache layer base, V cache layer base; else out[0]
  const float* bias[3];   // qkv bias (Qwen2) or nullptr
  const float* resid;     // kEpiResid: residual input; nullptr: embedding row of the token
};

struct PAttn {
  float* kcache;       // layer base [seq_len][kv_dim]
  const float* vcache;
  const float* qn;     // per-head q / k RMSNorm weights (Qwen3) or nullptr
  const float* kn;
};

struct PStepState {
  int32_t pos;         // position processed by the next launch
  int32_t token;       // token embedded by the next launch
  int32_t prompt_len;  // positions < prompt_len - 1 take their successor from the prompt
  int32_t sampled;     // argmax of the last sampled logits
};

struct PArgs {
  const PGemv* ph;     // [4 * L + 1]: per layer qkv, wo, w13, w2; then the classifier
  const PAttn* at;     // [L]
  int L, D, Dq, Dkv, V, S, kv_mul, KVH;
  float eps, qk_eps, scale;
  int rope_style, transform;
  const float* sin_t;
  const float* cos_t;
  const float* emb;
  const float* q;      // query [Dq] (QKV phase output)
  float* att;          // attention output [Dq]
  float* attn_part;    // split partials [KVH][G][kv_mul][HD + 2]
  unsigned int* attn_cnt;  // [KVH] arrival counters, zero between phases
  int attn_G;          // chunk slots per kv head
  float* am_pv;        // [gridDim] argmax partials
  int* am_pi;
  unsigned int* am_cnt;    // argmax / end-of-step arrival counter
  unsigned int* bar;       // grid barrier arrival counter
  unsigned int* bar_base;  // counter value at the start of the next launch
  int* err;
  int red_off;         // LDS: the GEMV input vector at 0, row partials at red_off floats
  PStepState* st;
  const int32_t* prompt;
  int32_t* out_tokens;
  // Optional device-time trace (nullptr: off).  Slot-major [slot][workgroup]
  // of 100 MHz s_memrealtime ticks: slot 0 = kernel entry, slots 2k+1 / 2k+2 =
  // arrival at / release from grid barrier k, slot 2 * n_barriers + 1 = end of
  // the workgroup's last phase.
  unsigned long long* trace;
};


// ---------------------------------------------------------------------------
// Address spaces.  Phase descriptors are read through the constant address
// space (scalar loads into SGPRs); weights, activations and counters through
// the global address space, so every access is a global_* (not flat_*)
// instruction and waits only for the vector-memory counter.
// ---------------------------------------------------------------------------
#define KL_GAS __attribute__((address_space(1)))
#define KL_CAS __attribute__((address_space(4)))
typedef const KL_CAS PGemv* PGp;

__device__ __forceinline__ float g_ld(const float* p) {
  return __hip_atomic_load((KL_GAS float*)(p),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int g_ld(const int* p) {
  return __hip_atomic_load((KL_GAS int*)(p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned int g_ld(const unsigned int* p) {
  return __hip_atomic_load((KL_GAS unsigned int*)(p),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void g_st(float* p, float v) {
  __hip_atomic_store((KL_GAS float*)(p), v, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void g_st(int* p, int v) {
  __hip_atomic_store((KL_GAS int*)(p), v, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void g_st(unsigned int* p, unsigned int v) {
  __hip_atomic_store((KL_GAS unsigned int*)(p), v, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned int g_arrive(unsigned int* p) {
  return __hip_atomic_fetch_add((KL_GAS unsigned int*)(p), 1u, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
}
// Plain (non-coherent) global loads of read-only data.
template <class T>
__device__ __forceinline__ T g_rd(const T* p) {
  return *(const KL_GAS T*)(p);
}
template <class T>
__device__ __forceinline__ T g_stream(const T* p) {
  return __builtin_nontemporal_load((const KL_GAS T*)(p));
}

__device__ __forceinline__ void trace_mark(const PArgs& a, int slot) {
  if (a.trace && threadIdx.x == 0)
    a.trace[static_cast<size_t>(slot) * gridDim.x + blockIdx.x] = __builtin_amdgcn_s_memrealtime();
}

// Grid barrier; `target` is this launch's running arrival target, `nbar` the
// barrier's index within the launch (for the trace).
__device__ __forceinline__ void grid_sync(const PArgs& a, unsigned int& target, int& nbar) {
  target += gridDim.x;
  wait_mem();
  __syncthreads();
  trace_mark(a, 2 * nbar + 1);
  if (threadIdx.x == 0) {
    if (g_ld(a.err) == 0) {
      g_arrive(a.bar);
      for (int spins = 0;; ++spins) {
        const unsigned int c = g_ld(a.bar);
        if (static_cast<int>(c - target) >= 0) break;
        if ((spins & 255) == 255 && g_ld(a.err) != 0) break;
        if (spins >= kSpinLimit) {
          g_st(a.err, kDevErrBarrier);
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
  }
  trace_mark(a, 2 * nbar + 2);
  ++nbar;
  __syncthreads();
}

// Sum over the 512 threads of the workgroup; `red` holds >= kPWaves floats.
__device__ __forceinline__ float block_sum_p(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kPWaves; ++w) t += red[w];
  return t;
}

// Stages an activation vector into LDS (coherent loads unless it is constant
// data such as an embedding row), applying RMSNorm when `nw` is set:
// y = w * (x * (1 / sqrt(mean(x^2) + eps))) (kernels/cpu/rmsnorm_kernel.cpp:30-32).
// Ends with a workgroup barrier.
__device__ __forceinline__ void stage_vec(const float* src, bool coherent, const float* nw,
                                          float eps, int n, float* xs, float* red) {
  float ss = 0.f;
  for (int b0 = 0; b0 < n; b0 += kPThreads * 8) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = b0 + k * kPThreads + threadIdx.x;
      v[k] = i < n ? (coherent ? g_ld(src + i) : g_rd(src + i)) : 0.f;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = b0 + k * kPThreads + threadIdx.x;
      if (i < n) {
        xs[i] = v[k];
        ss += v[k] * v[k];
      }
    }
  }
  if (nw) {
    ss = block_sum_p(ss, red);
    const float r = 1.f / sqrtf(ss / static_cast<float>(n) + eps);
    for (int i = threadIdx.x; i < n; i += kPThreads) xs[i] = g_rd(nw + i) * (r * xs[i]);
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// GEMV streaming.
// ---------------------------------------------------------------------------
template <bool Q8>
struct PItem;
template <>
struct PItem<false> {
  f4 w;
};
template <>
struct PItem<true> {
  i4 w;
  float s;
};

// This workgroup's share of a phase and this wave's item geometry.
struct PGeom {
  int base;  // first split-dimension row of the workgroup
  int cnt;   // split-dimension rows of the workgroup
  int nloc;  // local rows (paired: cnt per sub-matrix)
  int n_items;
  int rg, ksi;
};

__device__ __forceinline__ PGeom p_geom(PGp p) {
  PGeom g;
  // The wave index is uniform across the wave; readfirstlane lets the compiler
  // keep every item's row/sub-matrix arithmetic (and the descriptor loads it
  // drives) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  g.ksi = wave % p->ks;
  g.rg = wave / p->ks;
  const int total = p->paired ? p->rows[0] : p->rows[0] + p->rows[1] + p->rows[2];
  g.base = blockIdx.x * p->rpw;
  g.cnt = max(0, min(p->rpw, total - g.base));
  g.nloc = p->paired ? g.cnt * p->nsub : g.cnt;
  const int nrows = g.nloc > g.rg ? (g.nloc - g.rg + p->rw - 1) / p->rw : 0;
  g.n_items = nrows * p->nck;
  return g;
}

// Local row -> (sub-matrix, row).
__device__ __forceinline__ void p_row(PGp p, const PGeom& g, int lr, int& sub, int& row) {
  if (p->paired) {
    sub = 0;
    row = lr;
    while (row >= g.cnt) {
      row -= g.cnt;
      ++sub;
    }
    row += g.base;
  } else {
    int r = g.base + lr;
    sub = 0;
    if (r >= p->rows[0]) {
      r -= p->rows[0];
      sub = 1;
      if (r >= p->rows[1]) {
        r -= p->rows[1];
        sub = 2;
      }
    }
    row = r;
  }
}

// Item cursor: j-th item of the wave = (jr-th row of the wave, jc-th chunk).
struct PCur {
  int j, jr, jc;
};

__device__ __forceinline__ void p_advance(PCur& c, int nck) {
  ++c.j;
  if (++c.jc == nck) {
    c.jc = 0;
    ++c.jr;
  }
}

// Issues the loads of NB items starting at cursor c (advanced past them).
// Every load is issued unconditionally (items past the wave's last one and
// lanes past the row's end read a clamped, valid address; p_compute masks
// them out), so the code is straight-line and the compiler can wait for each
// item with an exact vmcnt instead of draining every outstanding load.
template <bool Q8, int NB>
__device__ __forceinline__ void p_issue(PGp p, const PGeom& g, PCur& c, PItem<Q8> (&buf)[NB]) {
  const int lane = threadIdx.x & 63;
  const int nck = p->nck, rw = p->rw, ks = p->ks, cn = p->cn, cn16 = p->cn16, cols = p->cols;
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    const bool item_ok = c.j < g.n_items;
    int sub = 0, row = 0, chunk = 0;
    if (item_ok) {
      p_row(p, g, g.rg + rw * c.jr, sub, row);
      chunk = g.ksi + ks * c.jc;
    }
    const int u = chunk * kWave + lane;  // 16-byte unit within the row
    const int uc = (item_ok && chunk < cn && u < cn16) ? u : 0;
    if constexpr (Q8) {
      const size_t e = static_cast<size_t>(row) * cols + static_cast<size_t>(uc) * 16;
      const int8_t* wp = static_cast<const int8_t*>(p->w[sub]);
      buf[k].w = g_stream(reinterpret_cast<const i4*>(wp + e));
      buf[k].s = g_rd(p->sc[sub] + (e >> p->gshift));
    } else {
      const float* wp = static_cast<const float*>(p->w[sub]) + static_cast<size_t>(row) * cols;
      buf[k].w = g_stream(reinterpret_cast<const f4*>(wp) + uc);
    }
    p_advance(c, nck);
  }
}

template <bool Q8>
__device__ __forceinline__ float p_dot(const PItem<Q8>& it, const float* xs, int u) {
  if constexpr (Q8) {
    const f4* xc = reinterpret_cast<const f4*>(xs) + 4 * u;
    float q[16];
    unpack_i8x4(it.w.x, q);
    unpack_i8x4(it.w.y, q + 4);
    unpack_i8x4(it.w.z, q + 8);
    unpack_i8x4(it.w.w, q + 12);
    f4 p = xc[0] * f4{q[0], q[1], q[2], q[3]};
    p += xc[1] * f4{q[4], q[5], q[6], q[7]};
    p += xc[2] * f4{q[8], q[9], q[10], q[11]};
    p += xc[3] * f4{q[12], q[13], q[14], q[15]};
    return hsum(p) * it.s;
  } else {
    return hsum(it.w * reinterpret_cast<const f4*>(xs)[u]);
  }
}

// Consumes NB items starting at cursor c; a finished row's wave total goes to
// red[local row * ks + k-slice].  Masked lanes and items contribute through a
// select, never a branch around the load's use.
template <bool Q8, int NB>
__device__ __forceinline__ void p_compute(PGp p, const PGeom& g, PCur& c,
                                          const PItem<Q8> (&buf)[NB], const float* xs, float* red,
                                          float& acc) {
  const int lane = threadIdx.x & 63;
  const int nck = p->nck, rw = p->rw, ks = p->ks, cn = p->cn, cn16 = p->cn16;
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    const bool item_ok = c.j < g.n_items;
    const int chunk = g.ksi + ks * c.jc;
    const int u = chunk * kWave + lane;
    const bool ok = item_ok && chunk < cn && u < cn16;
    const float d = p_dot<Q8>(buf[k], xs, ok ? u : 0);
    acc += ok ? d : 0.f;
    if (item_ok && c.jc == nck - 1) {
      const float v = wave_sum(acc);
      if (lane == 0) red[(g.rg + rw * c.jr) * ks + g.ksi] = v;
      acc = 0.f;
    }
    p_advance(c, nck);
  }
}

// Runs the streaming loop of one phase.  On entry, buffer A holds (in flight)
// the wave's first NB items of p; on exit A holds (in flight) the first NB
// items of `pn` (when pn is set).  Only A is live outside this function, so
// the attention phase and the staging code have the registers of B to
// themselves.  Returns with LDS `red` holding every finished row of the
// workgroup (after a workgroup barrier).
template <bool Q8, int NB>
__device__ __forceinline__ void p_stream(PGp p, const PGeom& g, PGp pn, const PGeom& gn,
                                         PItem<Q8> (&A)[NB], const float* xs, float* red) {
  PItem<Q8> B[NB];
  const int nck = p->nck;
  const int nb = (g.n_items + NB - 1) / NB;
  PCur ci{NB, NB / nck, NB % nck};  // issue cursor: batch 1
  PCur cc{0, 0, 0};                  // compute cursor
  float acc = 0.f;
  auto next_phase = [&]() {
    if (pn) {
      PCur c0{0, 0, 0};
      p_issue<Q8, NB>(pn, gn, c0, A);
    }
  };
  for (int b = 0; b < nb; b += 2) {
    // batch b is in A
    if (b + 1 < nb) {
      p_issue<Q8, NB>(p, g, ci, B);
      p_compute<Q8, NB>(p, g, cc, A, xs, red, acc);
    } else {
      p_compute<Q8, NB>(p, g, cc, A, xs, red, acc);
      break;
    }
    // batch b + 1 is in B; A is free
    if (b + 2 < nb)
      p_issue<Q8, NB>(p, g, ci, A);
    else
      next_phase();
    p_compute<Q8, NB>(p, g, cc, B, xs, red, acc);
  }
  if (nb % 2 == 1 || nb == 0) next_phase();
  __syncthreads();
}

// Sum of the KS slices of local row lr.
__device__ __forceinline__ float p_row_total(int ks, const float* red, int lr) {
  float v = 0.f;
  for (int k = 0; k < ks; ++k) v += red[lr * ks + k];
  return v;
}

// ---------------------------------------------------------------------------
// Attention phase (semantics of kernels/cpu/mha_kernel.cpp:5-61, with the
// optional Qwen3 per-head q/k RMSNorm (model/qwen3.cpp:485-500) and RoPE
// (kernels/cpu/rope_kernel.cpp) applied first).  One item = (kv head, chunk
// of PT positions); items are spread over the workgroups; the last chunk of a
// kv head to finish merges the chunks.  LDS floats needed: attn_p_lds_floats.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int attn_p_rpp(int hd) { return kPThreads / (hd / 4); }

__host__ __device__ inline size_t attn_p_lds_floats(int hd, int kv_mul, int G) {
  const int pt = attn_chunk(hd);
  const size_t head = static_cast<size_t>(kv_mul) * hd + static_cast<size_t>(kv_mul) * pt + hd +
                      2 * kAttnMaxKvMul;
  const size_t pv = static_cast<size_t>(attn_p_rpp(hd)) * kv_mul * hd;
  const size_t merge = 2 * static_cast<size_t>(G) * kv_mul;
  return head + (pv > merge ? pv : merge);
}

template <int HD>
__device__ __forceinline__ void attn_p_phase(const PArgs& a, const PAttn* atp, int pos,
                                             float* lds) {
  constexpr int PT = attn_chunk(HD);
  constexpr int TPR = HD / 4;
  constexpr int RPP = attn_p_rpp(HD);
  constexpr int NP = PT / RPP;
  constexpr int HALF = HD / 2;
  static_assert(NP >= 1 && NP * RPP == PT, "chunk geometry");
  __shared__ int s_last;
  const KL_CAS PAttn* at = (const KL_CAS PAttn*)(atp);
  float* kcache = at->kcache;
  const float* vcache = at->vcache;
  const float* qn = at->qn;
  const float* kn = at->kn;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int sub = tid % TPR;
  const int rr = tid / TPR;
  const int kvm = a.kv_mul;
  const int n = pos + 1;
  const int nsplit = (n + PT - 1) / PT;
  const int items = a.KVH * nsplit;
  float* qs = lds;                      // [kvm][HD]
  float* sc = qs + kvm * HD;            // [kvm][PT]
  float* kp = sc + kvm * PT;            // [HD]
  float* ml = kp + HD;                  // [2 * kAttnMaxKvMul]
  float* red = ml + 2 * kAttnMaxKvMul;  // [RPP][kvm][HD]; merge: [nsplit][kvm][2]
  for (int it = blockIdx.x; it < items; it += gridDim.x) {
    const int g = it / nsplit;
    const int s = it - g * nsplit;
    const int t0 = s * PT;
    const int cnt = min(n - t0, PT);
    const bool own_pos = pos >= t0 && pos < t0 + cnt;

    // 1. The chunk's K and V rows into registers; row pos was written in this
    //    launch (QKV phase) and is read coherently.
    f4 kr[NP], vr[NP];
    {
      const size_t col = static_cast<size_t>(g) * HD + 4 * sub;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int tt = p * RPP + rr;
        const int t = t0 + (tt < cnt ? tt : 0);
        const size_t off = static_cast<size_t>(t) * a.Dkv + col;
        if (t == pos) {
          kr[p] = f4{g_ld(kcache + off), g_ld(kcache + off + 1), g_ld(kcache + off + 2),
                     g_ld(kcache + off + 3)};
          vr[p] = f4{g_ld(vcache + off), g_ld(vcache + off + 1), g_ld(vcache + off + 2),
                     g_ld(vcache + off + 3)};
        } else {
          kr[p] = g_rd(reinterpret_cast<const f4*>(kcache + off));
          vr[p] = g_rd(reinterpret_cast<const f4*>(vcache + off));
        }
      }
    }
    // 2. q of the group's heads (coherent), q norm + RoPE in LDS; K[pos] transform.
    for (int i = tid; i < kvm * HD; i += kPThreads)
      qs[i] = g_ld(a.q + static_cast<size_t>(g) * kvm * HD + i);
    __syncthreads();
    if (a.transform == 2) {
      for (int h = wave; h < kvm; h += kPWaves) {
        float ss = 0.f;
        for (int d = lane; d < HD; d += kWave) ss += qs[h * HD + d] * qs[h * HD + d];
        ss = wave_sum(ss);
        const float r = 1.f / sqrtf(ss / static_cast<float>(HD) + a.qk_eps);
        for (int d = lane; d < HD; d += kWave) qs[h * HD + d] = (r * qs[h * HD + d]) * g_rd(qn + d);
      }
      __syncthreads();
    }
    if (a.transform >= 1) {
      const float* srow = a.sin_t + static_cast<size_t>(pos) * HD;
      const float* crow = a.cos_t + static_cast<size_t>(pos) * HD;
      for (int p = tid; p < kvm * HALF; p += kPThreads) {
        const int h = p / HALF, j = p - h * HALF;
        const int i0 = a.rope_style ? h * HD + j : h * HD + 2 * j;
        const int i1 = a.rope_style ? i0 + HALF : i0 + 1;
        float v0 = qs[i0], v1 = qs[i1];
        rope_pair(v0, v1, g_rd(crow + 2 * j), g_rd(srow + 2 * j));
        qs[i0] = v0;
        qs[i1] = v1;
      }
      if (wave == 0 && own_pos) {
        float* krow = kcache + static_cast<size_t>(pos) * a.Dkv + static_cast<size_t>(g) * HD;
        constexpr int PPL = (HALF + kWave - 1) / kWave;
        float v0[PPL], v1[PPL];
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < PPL; ++k) {
          const int j = lane + k * kWave;
          if (j < HALF) {
            const int i0 = a.rope_style ? j : 2 * j;
            const int i1 = a.rope_style ? j + HALF : 2 * j + 1;
            v0[k] = g_ld(krow + i0);
            v1[k] = g_ld(krow + i1);
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
              x0 = (r * x0) * g_rd(kn + i0);
              x1 = (r * x1) * g_rd(kn + i1);
            }
            rope_pair(x0, x1, g_rd(crow + 2 * j), g_rd(srow + 2 * j));
            g_st(krow + i0, x0);
            g_st(krow + i1, x1);
            kp[i0] = x0;
            kp[i1] = x1;
          }
        }
      }
      __syncthreads();
      if (own_pos) {
#pragma unroll
        for (int p = 0; p < NP; ++p)
          if (t0 + p * RPP + rr == pos) kr[p] = reinterpret_cast<const f4*>(kp)[sub];
      }
    }

    // 3. Scores.
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
    // 4. Chunk softmax statistics, one wave per head.
    for (int h = wave; h < kvm; h += kPWaves) {
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
    // 5. o_h = sum_t p_h[t] V_t.
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
    float* outg = a.att + static_cast<size_t>(g) * kvm * HD;
    float* pg = a.attn_part + static_cast<size_t>(g) * a.attn_G * kvm * (HD + 2);
    for (int idx = tid; idx < kvm * HD; idx += kPThreads) {
      const int h = idx / HD, d = idx - h * HD;
      float o = 0.f;
      for (int k = 0; k < RPP; ++k) o += red[(static_cast<size_t>(k) * kvm + h) * HD + d];
      if (nsplit == 1) {
        g_st(outg + h * HD + d, o / ml[2 * h + 1]);
      } else {
        float* ps = pg + (static_cast<size_t>(s) * kvm + h) * (HD + 2);
        g_st(ps + d, o);
        if (d == 0) {
          g_st(ps + HD, ml[2 * h]);
          g_st(ps + HD + 1, ml[2 * h + 1]);
        }
      }
    }
    if (nsplit > 1) {
      wait_mem();
      __syncthreads();
      if (tid == 0) {
        const unsigned int prev = g_arrive(a.attn_cnt + g);
        s_last = prev == static_cast<unsigned int>(nsplit - 1) ? 1 : 0;
      }
      __syncthreads();
      if (s_last) {
        // 6. Merge the chunks of this kv head.
        float* mls = red;  // [nsplit][kvm][2]
        for (int i = tid; i < nsplit * kvm; i += kPThreads) {
          const float* pk = pg + static_cast<size_t>(i) * (HD + 2);
          mls[2 * i] = g_ld(pk + HD);
          mls[2 * i + 1] = g_ld(pk + HD + 1);
        }
        __syncthreads();
        for (int idx = tid; idx < kvm * HD; idx += kPThreads) {
          const int h = idx / HD, d = idx - h * HD;
          float M = -INFINITY;
          for (int k = 0; k < nsplit; ++k) M = fmaxf(M, mls[2 * (k * kvm + h)]);
          float L = 0.f, O = 0.f;
          for (int k = 0; k < nsplit; ++k) {
            const float w = expf(mls[2 * (k * kvm + h)] - M);
            L += mls[2 * (k * kvm + h) + 1] * w;
            O += g_ld(pg + (static_cast<size_t>(k) * kvm + h) * (HD + 2) + d) * w;
          }
          g_st(outg + h * HD + d, O / L);
        }
        if (tid == 0) g_st(a.attn_cnt + g, 0u);
      }
    }
    __syncthreads();  // LDS is reused by the next item
  }
}

// ---------------------------------------------------------------------------
// Epilogues of the QKV, residual and SwiGLU phases.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void p_epilogue(PGp p, const PGeom& g, const float* red, int pos,
                                           const float* emb_row) {
  const int ks = p->ks;
  const int epi = p->epi;
  if (epi == kEpiQkv) {
    for (int lr = threadIdx.x; lr < g.nloc; lr += kPThreads) {
      int sub, row;
      p_row(p, g, lr, sub, row);
      float v = p_row_total(ks, red, lr);
      const float* b = p->bias[sub];
      if (b) v = v + g_rd(b + row);
      float* dst = sub == 0 ? p->out[0] + row
                            : p->out[sub] + static_cast<size_t>(pos) * p->rows[1] + row;
      g_st(dst, v);
    }
  } else if (epi == kEpiResid) {
    const float* resid = p->resid;
    float* out = p->out[0];
    for (int lr = threadIdx.x; lr < g.nloc; lr += kPThreads) {
      const int row = g.base + lr;
      const float r = resid ? g_ld(resid + row) : g_rd(emb_row + row);
      g_st(out + row, r + p_row_total(ks, red, lr));
    }
  } else if (epi == kEpiSwiglu) {
    float* out = p->out[0];
    for (int lr = threadIdx.x; lr < g.cnt; lr += kPThreads) {
      const float a1 = p_row_total(ks, red, lr);
      const float a3 = p_row_total(ks, red, lr + g.cnt);
      // kernels/cpu/swiglu_kernel.cpp:21-22
      const float s = a1 * (1.0f / (1.0f + expf(-a1)));
      g_st(out + g.base + lr, s * a3);
    }
  }
}

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
template <bool Q8, int NB, int HD>
__global__ __launch_bounds__(kPThreads) void k_decode_persistent(PArgs a) {
  extern __shared__ __align__(16) float lds[];
  __shared__ float sred[2 * kPWaves];
  __shared__ int s_last;
  __shared__ float s_bv[kPWaves];
  __shared__ int s_bi[kPWaves];
  const PStepState st = *a.st;  // written by the previous launch
  const int pos = st.pos;
  const int token = st.token;
  if (pos < 0 || pos >= a.S || token < 0 || token >= a.V) {
    if (blockIdx.x == 0 && threadIdx.x == 0) g_st(a.err, kDevErrPos);
    return;
  }
  const bool sample = pos + 1 >= st.prompt_len;
  unsigned int target = g_rd(a.bar_base);
  int nbar = 0;
  trace_mark(a, 0);
  const float* emb_row = a.emb + static_cast<size_t>(token) * a.D;
  const PGp ph = (PGp)(a.ph);
  const int ncls = 4 * a.L;  // index of the classifier phase
  float* xs = lds;
  float* red = lds + a.red_off;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

  PItem<Q8> A[NB];
  {
    const PGeom g0 = p_geom(ph);
    PCur c0{0, 0, 0};
    p_issue<Q8, NB>(ph, g0, c0, A);
  }
  float bv = -INFINITY;
  int bi = INT_MAX;
  for (int k = 0; k <= ncls; ++k) {
    const PGp p = ph + k;
    const bool is_cls = k == ncls;
    // The next GEMV phase (its first loads are issued before the barrier).
    const PGp pn = k + 1 < ncls ? ph + k + 1 : (k + 1 == ncls && sample ? ph + ncls : nullptr);
    const PGeom g = p_geom(p);
    const PGeom gn = pn ? p_geom(pn) : PGeom{};
    const float* in = p->in;
    stage_vec(in ? in : emb_row, in != nullptr, p->norm, a.eps, p->cols, xs, sred);
    p_stream<Q8, NB>(p, g, pn, gn, A, xs, red);
    if (is_cls) {
      // Logits (plain stores, read by the host after the launch) and this
      // workgroup's (max, first index) pair (sampler/argmax_sampler.cpp:5-13).
      float* logits = p->out[0];
      const int ks = p->ks;
      for (int lr = threadIdx.x; lr < g.nloc; lr += kPThreads) {
        const float v = p_row_total(ks, red, lr);
        logits[g.base + lr] = v;
        argmax_merge(bv, bi, v, g.base + lr);
      }
      wave_argmax(bv, bi);
      if (lane == 0) {
        s_bv[wave] = bv;
        s_bi[wave] = bi;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        for (int w = 1; w < kPWaves; ++w) argmax_merge(bv, bi, s_bv[w], s_bi[w]);
        g_st(a.am_pv + blockIdx.x, bv);
        g_st(reinterpret_cast<int*>(a.am_pi) + blockIdx.x, bi);
      }
      break;
    }
    p_epilogue(p, g, red, pos, emb_row);
    if (!pn) break;  // last layer of a prompt position: no classifier
    grid_sync(a, target, nbar);
    if ((k & 3) == 0) {  // after QKV: attention of layer k / 4
      attn_p_phase<HD>(a, a.at + (k >> 2), pos, lds);
      grid_sync(a, target, nbar);
    }
  }

  // End of step: the last workgroup to arrive samples (or takes the next
  // prompt token) and advances the device state for the next launch.
  trace_mark(a, 2 * nbar + 1);
  wait_mem();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned int prev = g_arrive(a.am_cnt);
    s_last = prev == gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last) return;
  int next;
  if (sample) {
    bv = -INFINITY;
    bi = INT_MAX;
    for (int b = threadIdx.x; b < static_cast<int>(gridDim.x); b += kPThreads)
      argmax_merge(bv, bi, g_ld(a.am_pv + b), g_ld(reinterpret_cast<const int*>(a.am_pi) + b));
    wave_argmax(bv, bi);
    if (lane == 0) {
      s_bv[wave] = bv;
      s_bi[wave] = bi;
    }
    __syncthreads();
    for (int w = 1; w < kPWaves; ++w) argmax_merge(bv, bi, s_bv[w], s_bi[w]);
    next = bi;
  } else {
    next = g_rd(a.prompt + pos + 1);
  }
  if (threadIdx.x == 0) {
    if (next < 0 || next >= a.V) {
      g_st(a.err, kDevErrToken);
      next = 0;
    }
    PStepState ns = st;
    if (sample) {
      ns.sampled = next;
      a.out_tokens[pos] = next;
    }
    ns.token = next;
    ns.pos = pos + 1;
    *a.st = ns;
    *a.bar_base = target;
    g_st(a.am_cnt, 0u);
  }
}

}  // namespace kl
