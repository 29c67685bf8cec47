// Persistent decode step: one launch runs a whole token of the
// reference forward (model/llama3.cpp:146-166, :599-744; qwen2.cpp:205-225;
// qwen3.cpp:147-167) on every CU at once.
//
// Phases of one token:
//   per layer:  QKV GEMV -> attention -> WO GEMV -> W1/W3 GEMV -> W2 GEMV
//   then:       classifier GEMV + argmax (sampled positions only)
//
// Why persistent: a decode step of Llama-3.2-1B streams 4.9 GB of weights in
// 81 GEMV-shaped pieces, most of them 17-67 MB.  As separate kernels each pays
// a launch, a ramp-up and a drain, and the small ones never reach full HBM
// bandwidth.  Here the 81 phases follow each other inside one launch, and a
// workgroup starts a phase the moment its input vector is complete (no grid
// barrier), so the chip streams weights nearly continuously.  The phase's first
// weight loads are issued before its input is polled, so they are on their way
// during the hand-off.
//
// Dataflow hand-off, no grid barriers.  Every activation that crosses
// workgroups (q, the new K and V rows, the attention output, the residual
// stream after WO and after W2, the FFN hidden vector) is stored as 64-bit
// {value, tag} pairs with one agent-coherent (sc1) store; a consumer stages
// its input by loading the pairs coherently and re-polling the elements whose
// tag is not yet the current one.  The tag is unique per (launch, layer):
// epoch * 128 + layer + 1, with `epoch` carried from launch to launch in
// device memory.  One round trip (the producer's store, the consumer's load)
// replaces barrier + staging load.  Safety of reuse: every workgroup owns at
// least one row of every GEMV phase (the host caps the grid at the smallest
// phase's row count), so no workgroup can start a phase before every
// workgroup has finished the previous one; each tagged buffer is rewritten
// only every fifth phase, long after its last reader.
//
// Residual stream.  WO and W2 both produce the D rows of the residual stream
// with the same row split, so each workgroup keeps its own rows of x in LDS
// and the residual adds read nothing from memory.
//
// GEMV phases.  The split dimension (output rows) is cut into contiguous
// ranges, one per workgroup: balanced, or weighted by each workgroup's
// measured streaming speed (the host calibrates once per engine: on a given
// part some XCDs stream a few percent slower than others).  Inside the workgroup, KS waves share
// a row (split-K) and RW = 8 / KS row groups take rows round robin; the host
// planner picks KS per phase.  A wave's work is a list of items = (local row,
// 1 KiB column chunk): 64 lanes x 16 bytes (4 fp32 or 16 int8 weights per
// lane), streamed through two register buffers of NB items (double
// buffering); a finished row's partial is reduced across the wave (DPP) and
// stored to LDS slot [row][k-slice], so the sum order is fixed and results are
// bitwise reproducible.
//
// Every wait is bounded: after kSpinLimit polls a workgroup records an error
// and every later wait of the launch returns at once, so every wave always
// reaches the end of the kernel; the host reports the error.
#pragma once
#include <math.h>

#include "attn.hpp"
#include "device.hpp"

namespace kl {

constexpr int kPThreads = 512;
constexpr int kPWaves = kPThreads / kWave;
constexpr int kSpinLimit = 1 << 22;
constexpr int kTagLayers = 128;  // tag = epoch * kTagLayers + layer + 1
// The epoch wraps to 0 after kEpochWrap launches, so tags stay below 2^31.
// Every tagged vector except the attention partials is rewritten by every
// launch, so its old tags never equal a new one; partial slots past a step's
// chunk count can sit untouched, so the wrapping launch zeroes them (tag 0 is
// never a valid tag).
constexpr unsigned int kEpochWrap = 1u << 24;

// Error codes written to PArgs::err by the device.
constexpr int kDevErrWait = 1;   // a wait for another workgroup exceeded kSpinLimit polls
constexpr int kDevErrPos = 2;    // position or token outside the model's range
constexpr int kDevErrToken = 3;  // the sampler found no finite maximum
constexpr int kDevErrVariant = 4;  // the launch's attention variant does not fit its position

enum : int { kEpiQkv = 0, kEpiResid = 1, kEpiSwiglu = 2, kEpiCls = 3 };

typedef unsigned long long tagged_t;  // {float bits (low), tag (high)}

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
  int ks, rw;             // waves per row (split-K), row groups; ks * rw == kPWaves
  int nseg;               // segments (NB consecutive chunks) per row
  int nsegw;              // segments per (row, wave) = ceil(nseg / ks)
  int epi;                // kEpi*
  int layer;              // tags: this phase writes tag(layer), reads tag(in_layer)
  int in_layer;
  const tagged_t* in;     // tagged input vector; nullptr: embedding row of the token
  const float* norm;      // RMSNorm weight applied to the input, or nullptr
  tagged_t* out[3];       // qkv: q, new K row, new V row; resid / swiglu: out[0]
  float* vcache;          // qkv: V cache layer base (row pos kept for later tokens)
  float* logits;          // classifier output
  const float* bias[3];   // qkv bias (Qwen2) or nullptr
  int dyn, blk;           // classifier: the last `dyn` rows are handed out at run time in
                          //   blocks of `blk` rows (0: every row in the static split)
  const int* split;       // [workgroups + 1] first row of each workgroup, or nullptr:
                          //   balanced split b * total / n
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
  const tagged_t* q;       // QKV phase outputs (tagged)
  const tagged_t* knew;
  const tagged_t* vnew;
  tagged_t* att;           // attention output [Dq] (tagged)
  tagged_t* attn_part;     // split partials [KVH][G][kv_mul][HD + 2] (tagged)
  long long attn_part_n;   // its elements
  int attn_G;              // chunk slots per kv head
  int merge_chunks;        // chunks per merging workgroup beyond 2 kAttnMergeChunks chunks
  int merge_chunks_mid;    //   and from kAttnMergeChunks + 1 to 2 kAttnMergeChunks chunks
  // Workgroups without an attention item pull the first w13_touch_rows local
  // rows of their W1/W3 share (0: none) into L2 while the attention runs,
  // after touch_delay 100 MHz ticks, and a slice of the attention
  // workgroups' rows.
  int touch_delay, w13_touch_rows;
  // Attention over at most attn_short_max positions (pos + 1) takes the
  // short-context path: one item per query head, no split (0: never).  Its
  // idle workgroups pull short_touch_rows local rows of W1/W3 into L2.
  int attn_short_max, short_touch_rows;
  int stage_pair_min;  // inputs at least this wide are staged in pairs
  // Its per-layer operands by arithmetic (no descriptor load on the critical
  // path): K/V cache layer l at kc0 / vc0 + l * kv_layer, Qwen3 q/k norm
  // weights at qkn + l * 2 * HD (q) and + HD (k).
  float* kc0;
  const float* vc0;
  long long kv_layer;
  const float* qkn;
  float* am_pv;            // [gridDim] argmax partials
  int* am_pi;
  unsigned int* am_cnt;    // end-of-step arrival counter
  unsigned int* cls_next;  // next dynamic classifier block (reset by the last workgroup)
  unsigned int* epoch;     // launch counter for tags
  int* err;
  int red_off;             // LDS floats: input vector at 0, row partials at red_off,
  int xres_off;            //   own residual rows at xres_off
  PStepState* st;
  const int32_t* prompt;
  int32_t* out_tokens;
  // Optional device-time trace (nullptr: off).  Slot-major [slot][workgroup]
  // of 100 MHz s_memrealtime ticks: slot 0 = kernel entry; phase p (5 per
  // layer: QKV, attention, WO, W1/W3, W2; then the classifier) has slot 2p+1 =
  // its input staged and slot 2p+2 = its outputs stored.  The marks are kept
  // in LDS (trace_slots 8-byte slots at u64 offset trace_off of the dynamic
  // LDS) and written out once at the end: a global store per mark would
  // perturb what it measures, because the vector-memory counter retires loads
  // and stores in order, so every later load wait would include the store's
  // acknowledgement.
  unsigned long long* trace;
  int trace_off, trace_slots;
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

__device__ __forceinline__ unsigned long long g_ld64(const tagged_t* p) {
  return __hip_atomic_load((KL_GAS tagged_t*)(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void g_st_tagged(tagged_t* p, float v, unsigned int tag) {
  const tagged_t x = (static_cast<tagged_t>(tag) << 32) | __float_as_uint(v);
  __hip_atomic_store((KL_GAS tagged_t*)(p), x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned int tag_of(tagged_t x) { return static_cast<unsigned int>(x >> 32); }
__device__ __forceinline__ float val_of(tagged_t x) {
  return __uint_as_float(static_cast<unsigned int>(x));
}

__device__ __forceinline__ unsigned long long* trace_lds(const PArgs& a) {
  extern __shared__ __align__(16) unsigned long long p_dyn_lds_u64[];
  return p_dyn_lds_u64 + a.trace_off;
}
__device__ __forceinline__ void trace_mark(const PArgs& a, int slot) {
  if (a.trace && threadIdx.x == 0) trace_lds(a)[slot] = __builtin_amdgcn_s_memrealtime();
}

// Re-polls, all together, the elements k of `v` (E values already loaded once
// from addr(k), valid where bit k of `valid` is set) that do not yet carry
// `tag`, until every one does: one round trip per retry however many are
// stale.  Bounded: after kSpinLimit retries (or once another workgroup has
// reported an error) it records the error and returns with what it holds.
template <int E, class Addr>
__device__ __forceinline__ void poll_many(const PArgs& a, unsigned int tag, Addr addr,
                                          unsigned int valid, tagged_t (&v)[E]) {
  unsigned int pend = 0;
#pragma unroll
  for (int k = 0; k < E; ++k)
    if (((valid >> k) & 1u) && tag_of(v[k]) != tag) pend |= 1u << k;
  for (int spins = 0; pend != 0; ++spins) {
    if ((spins & 63) == 63 && g_ld(a.err) != 0) break;
    if (spins >= kSpinLimit) {
      g_st(a.err, kDevErrWait);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int k = 0; k < E; ++k)
      if ((pend >> k) & 1u) v[k] = g_ld64(addr(k));
#pragma unroll
    for (int k = 0; k < E; ++k)
      if (((pend >> k) & 1u) && tag_of(v[k]) == tag) pend &= ~(1u << k);
  }
}

// The RMSNorm scale of a staged vector: 1 / sqrt(mean(x^2) + eps) from the
// per-wave sums of squares stage_vec left in ssq (after its barrier).
__device__ __forceinline__ float norm_scale(const float* ssq, int n, float eps) {
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kPWaves; ++w) t += ssq[w];
  return 1.f / sqrtf(t / static_cast<float>(n) + eps);
}

// Two adjacent tagged elements in one 16-byte device-coherent load (sc1, as
// the 8-byte atomic loads): twice the bytes per request, so a staged vector
// arrives in half the round trips.  Each element was written by one 8-byte
// store and carries its own tag, so a pair may hold one fresh and one stale
// element; the stale one is polled again.  Offsets past the buffer's
// `bytes` read zeros (tag 0: never a live tag).
struct tagged2 {
  tagged_t lo, hi;
};
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tagged_rsrc(const tagged_t* base, unsigned int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<tagged_t*>(base), static_cast<short>(0), bytes,
                                           0x00020000);
}
__device__ __forceinline__ tagged2 g_ld_pair(__amdgpu_buffer_rsrc_t r, int pair) {
  constexpr int kSc1 = 16;  // cache policy: device scope, as the 8-byte atomic loads
  const i4 v = __builtin_amdgcn_raw_buffer_load_b128(r, pair * 16, 0, kSc1);
  tagged2 t;
  t.lo = (static_cast<tagged_t>(static_cast<unsigned int>(v.y)) << 32) | static_cast<unsigned int>(v.x);
  t.hi = (static_cast<tagged_t>(static_cast<unsigned int>(v.w)) << 32) | static_cast<unsigned int>(v.z);
  return t;
}

// Stages a GEMV input vector into LDS: the tagged vector `src` (all n elements
// polled until they carry `tag`), or the embedding row `emb_row` when src is
// null.  With RMSNorm (`nw` set), y = w * (x * r), r = 1 / sqrt(mean(x^2) + eps)
// (kernels/cpu/rmsnorm_kernel.cpp:30-32), the staged vector is w * x and the
// scalar r is applied to the GEMV's row totals (W y = r (W (w * x))): the
// per-wave sums of squares go to ssq[kPWaves] and norm_scale() combines them
// after the closing barrier, so the norm adds no barrier or extra pass over
// the vector to the hand-off.  Each thread takes 8 elements per round.
// The phase's first weight segment is already in flight when the polling
// starts (the polls' answers wait for it: loads return in order).  Measured on
// Llama-3.2-1B with the short-context attention: +1.6% against issuing it
// after the staging (with the chunked attention and its merge hand-off the
// same change had measured -1.5%).
// Ends with a workgroup barrier.
//
// Layout in LDS: element i at i (fp32 weights: a lane reads 4 consecutive
// elements, lanes 16 bytes apart) or, PAD (int8 weights: a lane reads the 16
// elements of its 16 weights, lanes 64 bytes apart), at xpad(i) = i + 4 (i / 16):
// the 16 lanes of a quarter-wave 16-byte read then start 80 bytes apart and
// hit distinct banks.
__host__ __device__ constexpr int xpad(int i) { return i + ((i >> 4) << 2); }
template <bool PAD>
__device__ __forceinline__ void stage_vec_single(const PArgs& a, const tagged_t* src,
                                                 unsigned int tag, const float* emb_row,
                                                 const float* nw, int n, float* xs, float* ssq) {
  constexpr int T = kPThreads;
  const int tid = threadIdx.x;
  float ss = 0.f;
  float wv[8];  // norm weights of the first round
  for (int b0 = 0; b0 < n; b0 += T * 8) {
    tagged_t v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = b0 + k * T + tid;
      if (src)
        v[k] = i < n ? g_ld64(src + i) : (static_cast<tagged_t>(tag) << 32);
      else
        v[k] = (static_cast<tagged_t>(tag) << 32) | __float_as_uint(i < n ? g_rd(emb_row + i) : 0.f);
    }
    if (b0 == 0 && nw) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int i = k * T + tid;
        wv[k] = g_rd(nw + (i < n ? i : 0));
      }
    }
    if (src) {
      unsigned int valid = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (b0 + k * T + tid < n) valid |= 1u << k;
      poll_many<8>(a, tag, [&](int k) { return src + b0 + k * T + tid; }, valid, v);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = b0 + k * T + tid;
      if (i < n) {
        const float x = val_of(v[k]);
        ss += x * x;
        xs[PAD ? xpad(i) : i] = nw ? (b0 == 0 ? wv[k] : g_rd(nw + i)) * x : x;
      }
    }
  }
  if (nw) {
    ss = wave_sum(ss);
    if ((tid & 63) == 0) ssq[tid >> 6] = ss;
  }
  __syncthreads();
}

// stage_vec_single with two adjacent elements per load (n even): each thread
// takes 8 pairs per round, and a pair with a stale element is polled again.
template <bool PAD>
__device__ __forceinline__ void stage_vec_pairs(const PArgs& a, const tagged_t* src,
                                                unsigned int tag, const float* emb_row,
                                                const float* nw, int n, float* xs, float* ssq) {
  constexpr int T = kPThreads;
  constexpr int E = 8;  // pairs per thread per round
  const int tid = threadIdx.x;
  const int np = n >> 1;
  const tagged_t live = static_cast<tagged_t>(tag) << 32;
  const __amdgpu_buffer_rsrc_t r = tagged_rsrc(src, static_cast<unsigned int>(n) * 8u);
  float ss = 0.f;
  f2 wv[E];  // norm weights of the first round
  for (int b0 = 0; b0 < np; b0 += T * E) {
    tagged2 v[E];
#pragma unroll
    for (int k = 0; k < E; ++k) {
      const int i = b0 + k * T + tid;
      if (src) {
        v[k] = i < np ? g_ld_pair(r, i) : tagged2{live, live};
      } else {
        const f2 e = i < np ? g_rd(reinterpret_cast<const f2*>(emb_row) + i) : f2{0.f, 0.f};
        v[k] = tagged2{live | __float_as_uint(e.x), live | __float_as_uint(e.y)};
      }
    }
    if (b0 == 0 && nw) {
#pragma unroll
      for (int k = 0; k < E; ++k) {
        const int i = k * T + tid;
        wv[k] = g_rd(reinterpret_cast<const f2*>(nw) + (i < np ? i : 0));
      }
    }
    if (src) {
      // Pairs holding a stale element are polled again, all together, until
      // both carry the tag (bounded as poll_many).
      unsigned int pend = 0;
#pragma unroll
      for (int k = 0; k < E; ++k)
        if (tag_of(v[k].lo) != tag || tag_of(v[k].hi) != tag) pend |= 1u << k;
      for (int spins = 0; pend != 0; ++spins) {
        if ((spins & 63) == 63 && g_ld(a.err) != 0) break;
        if (spins >= kSpinLimit) {
          g_st(a.err, kDevErrWait);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < E; ++k)
          if ((pend >> k) & 1u) v[k] = g_ld_pair(r, b0 + k * T + tid);
#pragma unroll
        for (int k = 0; k < E; ++k)
          if (((pend >> k) & 1u) && tag_of(v[k].lo) == tag && tag_of(v[k].hi) == tag) pend &= ~(1u << k);
      }
    }
#pragma unroll
    for (int k = 0; k < E; ++k) {
      const int i = b0 + k * T + tid;
      if (i < np) {
        const float x0 = val_of(v[k].lo), x1 = val_of(v[k].hi);
        ss += x0 * x0;
        ss += x1 * x1;
        f2 y{x0, x1};
        if (nw) {
          const f2 w = b0 == 0 ? wv[k] : g_rd(reinterpret_cast<const f2*>(nw) + i);
          y = f2{w.x * x0, w.y * x1};
        }
        *reinterpret_cast<f2*>(xs + (PAD ? xpad(2 * i) : 2 * i)) = y;  // one 16-group
      }
    }
  }
  if (nw) {
    ss = wave_sum(ss);
    if ((tid & 63) == 0) ssq[tid >> 6] = ss;
  }
  __syncthreads();
}

// Inputs of at least a.stage_pair_min elements are staged in pairs (half the
// round trips); narrower ones one element per load, which measured faster
// for the 2048-wide inputs of Llama-3.2-1B and the 768-wide ones of
// Llama2-110M (where each thread holds only a few elements).
template <bool PAD>
__device__ __forceinline__ void stage_vec(const PArgs& a, const tagged_t* src, unsigned int tag,
                                          const float* emb_row, const float* nw, int n, float* xs,
                                          float* ssq) {
  if (n >= a.stage_pair_min)
    stage_vec_pairs<PAD>(a, src, tag, emb_row, nw, n, xs, ssq);
  else
    stage_vec_single<PAD>(a, src, tag, emb_row, nw, n, xs, ssq);
}

// Lane-shifted copy of x through DPP (lanes without a source read 0).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_shift(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, false));
}

// Sum over the 64 lanes with DPP row shifts and row broadcasts; the total is
// valid in lane 63 only.
__device__ __forceinline__ float wave_sum_to_63(float v) {
  v += dpp_shift<0x111, 0xf>(v);  // row_shr:1
  v += dpp_shift<0x112, 0xf>(v);  // row_shr:2
  v += dpp_shift<0x114, 0xf>(v);  // row_shr:4
  v += dpp_shift<0x118, 0xf>(v);  // row_shr:8   -> lane 15 of each row holds the row sum
  v += dpp_shift<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_shift<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// Sum over aligned groups of W lanes (W in 8, 16, 32, 64) with DPP butterflies
// (quad_perm, half-row and row mirrors, row broadcasts): valid in lane W - 1
// of each group (W <= 16: in every lane of the group).
template <int W>
__device__ __forceinline__ float group_sum_dpp(float v) {
  static_assert(W == 8 || W == 16 || W == 32 || W == 64, "group width");
  v += dpp_shift<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
  v += dpp_shift<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
  v += dpp_shift<0x141, 0xf>(v);  // row_half_mirror: the two quads of each 8 lanes
  if (W >= 16) v += dpp_shift<0x140, 0xf>(v);  // row_mirror: the two halves of each row
  if (W >= 32) v += dpp_shift<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  if (W >= 64) v += dpp_shift<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// Maximum over the 64 lanes, returned to every lane (uniform).
__device__ __forceinline__ float wave_max_dpp(float v) {
  auto mx = [](float a, float b) { return fmaxf(a, b); };
  // -inf as the neutral element: shifted-in lanes read 0, so use mirrors and
  // broadcasts whose sources are always valid lanes.
  v = mx(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0xB1, 0xf, 0xf, false)));
  v = mx(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x4E, 0xf, 0xf, false)));
  v = mx(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x141, 0xf, 0xf, false)));
  v = mx(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x140, 0xf, 0xf, false)));
  v = mx(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x142, 0xa, 0xf, false)));
  v = mx(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x143, 0xc, 0xf, false)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum over the 64 lanes, returned to every lane (uniform).
__device__ __forceinline__ float wave_sum_dpp(float v) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(group_sum_dpp<64>(v)), 63));
}

// ---------------------------------------------------------------------------
// GEMV streaming.
//
// Unit of work: a segment = NB consecutive 1 KiB chunks of one row (64 lanes x
// 16 bytes per chunk: 4 fp32 or 16 int8 weights per lane).  A wave owns the
// segments (row rg + rw * jr, segment ksi + ks * js) of its workgroup's rows;
// per segment it issues NB loads from one scalar row pointer, so all
// bookkeeping is per segment, not per chunk.  Segments are double buffered in
// registers.  When every wave always reads the same segment of its rows
// (nsegw == 1), the matching slice of the fp32 input stays in registers for
// the whole phase instead of being read from LDS per chunk.
// ---------------------------------------------------------------------------
template <bool Q8>
struct PChunk;
template <>
struct PChunk<false> {
  f4 w;
};
template <>
struct PChunk<true> {
  i4 w;
  float s;
};

// This workgroup's share of a phase and this wave's segment geometry.
struct PGeom {
  int base;  // first split-dimension row of the workgroup
  int cnt;   // split-dimension rows of the workgroup
  int nloc;  // local rows (paired: cnt per sub-matrix)
  int n_items;  // segments of this wave
  int rg, ksi;
};

// Rows [base, base + cnt) of a phase owned by workgroup b.
__device__ __forceinline__ void p_share(PGp p, int b, int& base, int& cnt) {
  if (p->split) {
    // Measured split: rows in proportion to each workgroup's streaming speed.
    const KL_CAS int* sp = (const KL_CAS int*)(p->split);
    base = sp[b];
    cnt = sp[b + 1] - base;
  } else {
    // Balanced split: workgroup b owns rows [b * total / n, (b + 1) * total / n)
    // of the statically split rows.
    const int total = (p->paired ? p->rows[0] : p->rows[0] + p->rows[1] + p->rows[2]) - p->dyn;
    const long long bb = b, n = gridDim.x;
    base = static_cast<int>(bb * total / n);
    cnt = static_cast<int>((bb + 1) * total / n) - base;
  }
}

__device__ __forceinline__ PGeom p_geom(PGp p) {
  PGeom g;
  // The wave index is uniform across the wave; readfirstlane lets the compiler
  // keep every segment's row/sub-matrix arithmetic (and the descriptor loads it
  // drives) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  g.ksi = wave % p->ks;
  g.rg = wave / p->ks;
  p_share(p, blockIdx.x, g.base, g.cnt);
  g.nloc = p->paired ? g.cnt * p->nsub : g.cnt;
  const int nrows = g.nloc > g.rg ? (g.nloc - g.rg + p->rw - 1) / p->rw : 0;
  g.n_items = g.ksi < p->nseg ? nrows * p->nsegw : 0;
  return g;
}

// Geometry of dynamic classifier block `blk`: rows [v0 + blk * B, + B) of the
// rows past the static split (v0 = total - dyn), clipped to the matrix.
__device__ __forceinline__ PGeom p_geom_block(PGp p, int blk) {
  PGeom g;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  g.ksi = wave % p->ks;
  g.rg = wave / p->ks;
  const int first = p->rows[0] - p->dyn + blk * p->blk;
  g.base = first;
  g.cnt = min(p->blk, p->rows[0] - first);
  g.nloc = g.cnt;
  const int nrows = g.nloc > g.rg ? (g.nloc - g.rg + p->rw - 1) / p->rw : 0;
  g.n_items = g.ksi < p->nseg ? nrows * p->nsegw : 0;
  return g;
}

// A byte range of weight rows to pull into L2, in 128-byte lines.
struct TouchSpan {
  const char* ptr;
  int lines;
};

// Local rows [r0, r1) of workgroup b's share of a paired phase (rows of its
// first sub-matrix; r1 is clipped to the share): weights in w, int8 scales in
// sc (empty for fp32).
template <bool Q8>
__device__ __forceinline__ void p_touch_rows(PGp p, int b, int r0, int r1, TouchSpan& w,
                                             TouchSpan& sc) {
  int base, cnt;
  p_share(p, b, base, cnt);
  r1 = min(r1, cnt);
  const size_t e0 = static_cast<size_t>(base + r0) * p->cols;
  const size_t ne = r1 > r0 ? static_cast<size_t>(r1 - r0) * p->cols : 0;
  w.ptr = static_cast<const char*>(p->w[0]) + e0 * (Q8 ? 1 : 4);
  w.lines = static_cast<int>((ne * (Q8 ? 1 : 4) + 127) / 128);
  sc.ptr = w.ptr;
  sc.lines = 0;
  if constexpr (Q8) {
    sc.ptr = reinterpret_cast<const char*>(p->sc[0] + (e0 >> p->gshift));
    sc.lines = static_cast<int>(((ne >> p->gshift) * 4 + 127) / 128);
  }
}

// Reads one word of every 128-byte line of the spans (up to 8 lines per
// thread, all issued before any is waited for), so that the lines sit in this
// XCD's L2 when their phase streams them.  Returns an XOR of the words, which
// the caller keeps live.
__device__ __forceinline__ unsigned int p_touch_lines(TouchSpan s0, TouchSpan s1, TouchSpan s2,
                                                      TouchSpan s3, TouchSpan s4, TouchSpan s5) {
  const int total = s0.lines + s1.lines + s2.lines + s3.lines + s4.lines + s5.lines;
  if (total == 0) return 0;
  auto at = [&](int f) {
    if (f < s0.lines) return s0.ptr + static_cast<size_t>(f) * 128;
    f -= s0.lines;
    if (f < s1.lines) return s1.ptr + static_cast<size_t>(f) * 128;
    f -= s1.lines;
    if (f < s2.lines) return s2.ptr + static_cast<size_t>(f) * 128;
    f -= s2.lines;
    if (f < s3.lines) return s3.ptr + static_cast<size_t>(f) * 128;
    f -= s3.lines;
    if (f < s4.lines) return s4.ptr + static_cast<size_t>(f) * 128;
    f -= s4.lines;
    return s5.ptr + static_cast<size_t>(f) * 128;
  };
  unsigned int v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int f = static_cast<int>(threadIdx.x) + k * kPThreads;
    v[k] = g_rd(reinterpret_cast<const unsigned int*>(at(f < total ? f : 0)));
  }
  unsigned int acc = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) acc ^= v[k];
  return acc;
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

// Segment cursor: j-th segment of the wave = (jr-th row of the wave, js-th
// segment of that row).
struct PCur {
  int j, jr, js;
};

__device__ __forceinline__ void p_advance(PCur& c, int nsegw) {
  ++c.j;
  if (++c.js == nsegw) {
    c.js = 0;
    ++c.jr;
  }
}

// Issues the NB loads of the segment at cursor c (then advances it).  Every
// load is issued (a wave without a segment left reads a clamped valid
// address, lanes past the row's end read the row start; p_seg_compute masks
// both), so the code is straight-line and each use waits with an exact vmcnt.
template <bool Q8, int NB>
__device__ __forceinline__ void p_seg_issue(PGp p, const PGeom& g, PCur& c,
                                            PChunk<Q8> (&buf)[NB]) {
  const int lane = threadIdx.x & 63;
  const bool item_ok = c.j < g.n_items;
  int sub = 0, row = 0, seg = 0;
  if (item_ok) {
    p_row(p, g, g.rg + p->rw * c.jr, sub, row);
    seg = g.ksi + p->ks * c.js;
  }
  const int lim = item_ok ? p->cn16 : 0;  // valid 16-byte units of the row
  const int u0 = seg * NB * kWave + lane;
  const int cols = p->cols;
  if constexpr (Q8) {
    const size_t e0 = static_cast<size_t>(row) * cols;
    const int8_t* wp = static_cast<const int8_t*>(p->w[sub]) + e0;
    // Rows hold whole groups (cols is a multiple of the group size, a power
    // of two of at least 16), so chunk u of the row has scale u >> cshift.
    const float* sp = p->sc[sub] + (e0 >> p->gshift);
    const int cshift = p->gshift - 4;
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int u = u0 + k * kWave;
      const int uc = u < lim ? u : 0;
      buf[k].w = g_stream(reinterpret_cast<const i4*>(wp) + uc);
      buf[k].s = g_rd(sp + (uc >> cshift));
    }
  } else {
    const f4* wp = reinterpret_cast<const f4*>(static_cast<const float*>(p->w[sub]) +
                                               static_cast<size_t>(row) * cols);
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int u = u0 + k * kWave;
      buf[k].w = g_stream(wp + (u < lim ? u : 0));
    }
  }
  p_advance(c, p->nsegw);
}

template <bool Q8>
__device__ __forceinline__ float p_dot(const PChunk<Q8>& it, const float* xs, int u) {
  if constexpr (Q8) {
    const f4* xc = reinterpret_cast<const f4*>(xs + xpad(16 * u));  // the padded layout
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

// Consumes the segment at cursor c; a finished row's wave total goes to
// red[local row * ks + k-slice].  xr holds the wave's input slice when xreg.
template <bool Q8, int NB>
__device__ __forceinline__ void p_seg_compute(PGp p, const PGeom& g, PCur& c,
                                              const PChunk<Q8> (&buf)[NB], const float* xs,
                                              const f4 (&xr)[NB], bool xreg, float* red,
                                              float& acc) {
  const int lane = threadIdx.x & 63;
  const bool item_ok = c.j < g.n_items;
  const int seg = g.ksi + p->ks * c.js;
  const int lim = item_ok ? p->cn16 : 0;
  const int u0 = seg * NB * kWave + lane;
  float part = 0.f;
  if (!Q8 && xreg) {
    f4 a4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const f4 prod = reinterpret_cast<const f4&>(buf[k].w) * xr[k];
      a4 += (u0 + k * kWave) < lim ? prod : f4{0.f, 0.f, 0.f, 0.f};
    }
    part = hsum(a4);
  } else {
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int u = u0 + k * kWave;
      const bool ok = u < lim;
      const float d = p_dot<Q8>(buf[k], xs, ok ? u : 0);
      part += ok ? d : 0.f;
    }
  }
  acc += part;
  if (item_ok && c.js == p->nsegw - 1) {
    const float v = wave_sum_to_63(acc);
    if (lane == 63) red[(g.rg + p->rw * c.jr) * p->ks + g.ksi] = v;
    acc = 0.f;
  }
  p_advance(c, p->nsegw);
}

// Runs the streaming loop of one phase.  On entry, buffer A holds (in flight)
// the wave's first segment of p; B is the second buffer.  Only A is live
// outside this function.  Returns with LDS `red` holding every finished row
// of the workgroup (after a workgroup barrier).
template <bool Q8, int NB>
__device__ __forceinline__ void p_stream(PGp p, const PGeom& g, PChunk<Q8> (&A)[NB],
                                         const float* xs, float* red) {
  PChunk<Q8> B[NB];
  const int nb = g.n_items;
  PCur ci{1, 1 / p->nsegw, 1 % p->nsegw};  // issue cursor: segment 1
  PCur cc{0, 0, 0};                          // compute cursor
  // The wave's input slice in registers when it always reads one segment.
  const bool xreg = !Q8 && p->nsegw == 1;
  f4 xr[NB];
  if (!Q8) {
    const int u0 = g.ksi * NB * kWave + (threadIdx.x & 63);
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int u = u0 + k * kWave;
      xr[k] = xreg && u < p->cn16 ? reinterpret_cast<const f4*>(xs)[u] : f4{0.f, 0.f, 0.f, 0.f};
    }
  }
  float acc = 0.f;
  // Every step issues the next segment into the buffer computed in the step
  // before, then consumes the other.  Issues are unconditional (past the
  // wave's last segment they read one clamped valid address and are never
  // consumed), so each consume waits with an exact vmcnt.
  // The two loop shapes differ in one respect.  With the exit in the middle
  // (fp32), the compiler's merged exit block is also a path back to the loop
  // head on which buffer B is still in flight, so each iteration starts with
  // a full drain (vmcnt(0)) and at most one segment is in flight there.  With
  // the exit at the head (int8), both buffers stay in flight.  Measured: the
  // deeper int8 stream is 1.2% faster on Llama2-7B int8; the same shape for
  // fp32 slows the W1/W3 stream of Llama-3.2-1B by 7% (more requests in flight
  // per CU than HBM serves well when each wave streams its own rows).
  if constexpr (Q8) {
    int b = 0;
    for (; b + 1 < nb; b += 2) {
      p_seg_issue<Q8, NB>(p, g, ci, B);
      p_seg_compute<Q8, NB>(p, g, cc, A, xs, xr, xreg, red, acc);
      p_seg_issue<Q8, NB>(p, g, ci, A);
      p_seg_compute<Q8, NB>(p, g, cc, B, xs, xr, xreg, red, acc);
    }
    if (b < nb) p_seg_compute<Q8, NB>(p, g, cc, A, xs, xr, xreg, red, acc);
  } else {
    for (int b = 0; b < nb; b += 2) {
      p_seg_issue<Q8, NB>(p, g, ci, B);
      p_seg_compute<Q8, NB>(p, g, cc, A, xs, xr, xreg, red, acc);
      if (b + 1 >= nb) break;
      p_seg_issue<Q8, NB>(p, g, ci, A);
      p_seg_compute<Q8, NB>(p, g, cc, B, xs, xr, xreg, red, acc);
    }
  }
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
// of PT positions); items are spread over the workgroups; every chunk writes
// its partial (o, m, l) as tagged values, and the workgroups of a kv head's
// chunks merge them, each a slice of the head's outputs.  Rows before pos come from the cache
// (written by earlier launches); q and the new K/V rows come from the tagged
// QKV outputs.  The chunk that holds pos writes the transformed K row to the
// cache for later tokens.  Inside a chunk: a row's K in registers (HD / 4
// lanes x float4), scores by 16-lane DPP sums, the heads of the group four at
// a time so the reductions overlap; V staged to LDS and o = p V summed by
// groups of 8 adjacent lanes, each group owning one float4 of the output.
// LDS floats needed: attn_p_lds_floats.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int attn_p_rpp(int hd) { return kPThreads / (hd / 4); }
constexpr int kAttnMergeChunks = 8;  // chunks per merging workgroup

// The chunk's V rows sit in LDS with a row stride of hd + 4 floats: the PV
// step's eight lanes per output read eight different rows of the same
// columns, which at a stride of hd floats (a multiple of the bank period) all
// hit the same banks.
__host__ __device__ constexpr int attn_vs_stride(int hd) { return hd + 4; }

__host__ __device__ inline size_t attn_p_lds_floats(int hd, int kv_mul) {
  const int pt = attn_chunk(hd);
  const size_t head = static_cast<size_t>(kv_mul) * hd + static_cast<size_t>(kv_mul) * pt +
                      2 * static_cast<size_t>(hd) + 2 * kAttnMaxKvMul;
  return head + static_cast<size_t>(pt) * attn_vs_stride(hd);  // + the chunk's V rows
}

// Per-lane elements of the Qwen3 q/k norm weights (HD values over 64 lanes).
template <int HD>
constexpr int kNormPerLane = HD >= kWave ? HD / kWave : 1;

template <int HD>
__device__ __forceinline__ void attn_p_phase(const PArgs& a, const PAttn* atp, int pos,
                                             unsigned int tag, float* lds, int trace_slot,
                                             float rope_c, float rope_s) {
  constexpr int PT = attn_chunk(HD);
  constexpr int TPR = HD / 4;
  constexpr int RPP = attn_p_rpp(HD);
  constexpr int NP = PT / RPP;
  constexpr int HALF = HD / 2;
  static_assert(NP >= 1 && NP * RPP == PT, "chunk geometry");
  const KL_CAS PAttn* at = (const KL_CAS PAttn*)(atp);
  float* kcache = at->kcache;
  const float* vcache = at->vcache;
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
  float* kp = sc + kvm * PT;            // [HD] K[pos] (transformed)
  float* vp = kp + HD;                  // [HD] V[pos]
  float* ml = vp + HD;                  // [2 * kAttnMaxKvMul]
  float* vs = ml + 2 * kAttnMaxKvMul;   // [PT][HD + 4] V rows of the chunk
  for (int it = blockIdx.x; it < items; it += gridDim.x) {
    const int g = it / nsplit;
    const int s = it - g * nsplit;
    const int t0 = s * PT;
    const int cnt = min(n - t0, PT);
    const bool own_pos = pos >= t0 && pos < t0 + cnt;

    // 1. The chunk's cached K and V rows into registers (row pos is replaced
    //    below by the new row), requested before the polls below so that they
    //    arrive with them.  (Prefetching them during the QKV phase put their
    //    bytes ahead of that phase's polls in each wave's in-order return
    //    queue, and its registers made the head-size-128 variant spill.)
    f4 kr[NP], vr[NP];
    {
      const size_t col = static_cast<size_t>(g) * HD + 4 * sub;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int tt = p * RPP + rr;
        const int t = t0 + (tt < cnt && t0 + tt != pos ? tt : 0);  // row pos comes from QKV
        const size_t off = static_cast<size_t>(t) * a.Dkv + col;
        kr[p] = g_rd(reinterpret_cast<const f4*>(kcache + off));
        vr[p] = g_rd(reinterpret_cast<const f4*>(vcache + off));
      }
    }
    // Qwen3 q/k norm weights: requested just before the polls below, so
    //    they arrive with them and are live only in this phase.
    float qn[kNormPerLane<HD>], kn[kNormPerLane<HD>];
#pragma unroll
    for (int k = 0; k < kNormPerLane<HD>; ++k) {
      const int d = lane + k * kWave;
      qn[k] = a.transform == 2 && d < HD ? g_rd(at->qn + d) : 0.f;
      kn[k] = a.transform == 2 && d < HD ? g_rd(at->kn + d) : 0.f;
    }
    // 2. q of the group's heads and (chunk of pos) the new K and V rows, polled
    //    together (element e < kvm * HD is q, the next 2 * HD are K then V).
    {
      const int nq = kvm * HD, ne = nq + (own_pos ? 2 * HD : 0);
      const tagged_t* qg = a.q + static_cast<size_t>(g) * kvm * HD;
      auto addr = [&](int e) -> const tagged_t* {
        if (e < nq) return qg + e;
        e -= nq;
        return (e < HD ? a.knew : a.vnew) + static_cast<size_t>(g) * HD + (e < HD ? e : e - HD);
      };
      for (int e0 = tid; e0 < ne; e0 += 4 * kPThreads) {
        tagged_t v[4];
        unsigned int valid = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int e = e0 + k * kPThreads;
          if (e < ne) valid |= 1u << k;
          v[k] = g_ld64(addr(e < ne ? e : 0));
        }
        poll_many<4>(a, tag, [&](int k) {
          const int e = e0 + k * kPThreads;
          return addr(e < ne ? e : 0);
        }, valid, v);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int e = e0 + k * kPThreads;
          if (e < nq) qs[e] = val_of(v[k]);
          else if (e < ne) kp[e - nq] = val_of(v[k]);  // kp, then vp
        }
      }
    }
    __syncthreads();
    if (it == static_cast<int>(blockIdx.x)) trace_mark(a, trace_slot);  // inputs arrived
    if (a.transform == 2) {
      for (int h = wave; h < kvm; h += kPWaves) {
        float ss = 0.f;
        for (int d = lane; d < HD; d += kWave) ss += qs[h * HD + d] * qs[h * HD + d];
        ss = wave_sum(ss);
        const float r = 1.f / sqrtf(ss / static_cast<float>(HD) + a.qk_eps);
#pragma unroll
        for (int k = 0; k < kNormPerLane<HD>; ++k) {
          const int d = lane + k * kWave;
          if (d < HD) qs[h * HD + d] = (r * qs[h * HD + d]) * qn[k];
        }
      }
      if (own_pos && wave == kPWaves - 1) {
        float ss = 0.f;
        for (int d = lane; d < HD; d += kWave) ss += kp[d] * kp[d];
        ss = wave_sum(ss);
        const float r = 1.f / sqrtf(ss / static_cast<float>(HD) + a.qk_eps);
#pragma unroll
        for (int k = 0; k < kNormPerLane<HD>; ++k) {
          const int d = lane + k * kWave;
          if (d < HD) kp[d] = (r * kp[d]) * kn[k];
        }
      }
      __syncthreads();
    }
    if (a.transform >= 1) {
      // Every pair this thread rotates has j = tid % HALF (512 is a multiple
      // of HALF), whose table entries rope_c / rope_s the kernel loaded once.
      const int heads = own_pos ? kvm + 1 : kvm;  // head kvm = the new K row
      for (int p = tid; p < heads * HALF; p += kPThreads) {
        const int h = p / HALF, j = p - h * HALF;
        float* v = h < kvm ? qs + h * HD : kp;
        const int i0 = a.rope_style ? j : 2 * j;
        const int i1 = a.rope_style ? j + HALF : 2 * j + 1;
        float v0 = v[i0], v1 = v[i1];
        rope_pair(v0, v1, rope_c, rope_s);
        v[i0] = v0;
        v[i1] = v1;
      }
      __syncthreads();
    }
    if (own_pos) {
      // The new rows join the chunk; K[pos] (transformed) goes to the cache.
      float* krow = kcache + static_cast<size_t>(pos) * a.Dkv + static_cast<size_t>(g) * HD;
      for (int d = tid; d < HD; d += kPThreads) krow[d] = kp[d];
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        if (t0 + p * RPP + rr == pos) {
          kr[p] = reinterpret_cast<const f4*>(kp)[sub];
          vr[p] = reinterpret_cast<const f4*>(vp)[sub];
        }
      }
    }

    // The chunk's V rows to LDS for step 5 (row-major [PT][HD]).
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int tt = p * RPP + rr;
      if (tt < PT) reinterpret_cast<f4*>(vs + static_cast<size_t>(tt) * attn_vs_stride(HD))[sub] = vr[p];
    }

    // 3. Scores, four heads at a time (the q reads and the 16-lane reductions
    //    of the four heads and NP rows are independent and overlap).
    {
      const f4* q4 = reinterpret_cast<const f4*>(qs);
      for (int h0 = 0; h0 < kvm; h0 += 4) {
        f4 qv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) qv[j] = q4[min(h0 + j, kvm - 1) * TPR + sub];
        float d[NP][4];
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int j = 0; j < 4; ++j) d[p][j] = hsum(kr[p] * qv[j]);
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int j = 0; j < 4; ++j) d[p][j] = group_sum_dpp<TPR>(d[p][j]);
        if (sub == TPR - 1) {
#pragma unroll
          for (int p = 0; p < NP; ++p) {
            const int tt = p * RPP + rr;
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (tt < cnt && h0 + j < kvm) sc[(h0 + j) * PT + tt] = d[p][j] * a.scale;
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
      m = wave_max_dpp(m);
      float l = 0.f;
      for (int tt = lane; tt < cnt; tt += kWave) {
        const float e = expf(sh[tt] - m);
        sh[tt] = e;
        l += e;
      }
      l = wave_sum_dpp(l);
      if (lane == 0) {
        ml[2 * h] = m;
        ml[2 * h + 1] = l;
      }
    }
    __syncthreads();
    // 5. o_h = sum_t p_h[t] V_t: each output float4 (head h, dims 4 sub4 ..)
    //    by PV_T adjacent lanes over PT / PV_T rows each, summed by DPP; the
    //    chunk's output (one chunk: o / l) or its partial (o, m, l) is stored
    //    by the first lane of each group.
    {
      constexpr int PV_T = 8;
      constexpr int RPT = PT / PV_T;
      static_assert(PT % PV_T == 0, "rows per lane");
      const f4* v4 = reinterpret_cast<const f4*>(vs);
      tagged_t* outg = a.att + static_cast<size_t>(g) * kvm * HD;
      tagged_t* pg = a.attn_part + static_cast<size_t>(g) * a.attn_G * kvm * (HD + 2);
      for (int b = tid; b < kvm * TPR * PV_T; b += kPThreads) {
        const int part = b & (PV_T - 1), o4 = b / PV_T;
        const int h = o4 / TPR, sub4 = o4 - h * TPR;
        const float* ph = sc + h * PT;
        // Straight-line over the lane's rows: every row of vs holds finite
        // values (rows past the chunk were loaded from its first row), and
        // their weight is 0.
        f4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
          const int tt = part * RPT + j;
          const float w = ph[tt];
          o += (tt < cnt ? w : 0.f) * v4[tt * (attn_vs_stride(HD) / 4) + sub4];
        }
        o.x = group_sum_dpp<PV_T>(o.x);
        o.y = group_sum_dpp<PV_T>(o.y);
        o.z = group_sum_dpp<PV_T>(o.z);
        o.w = group_sum_dpp<PV_T>(o.w);
        if (part == 0) {
          const int d = 4 * sub4;
          if (nsplit == 1) {
            const float l = ml[2 * h + 1];
            tagged_t* op = outg + h * HD + d;
            g_st_tagged(op + 0, o.x / l, tag);
            g_st_tagged(op + 1, o.y / l, tag);
            g_st_tagged(op + 2, o.z / l, tag);
            g_st_tagged(op + 3, o.w / l, tag);
          } else {
            tagged_t* ps = pg + (static_cast<size_t>(s) * kvm + h) * (HD + 2);
            g_st_tagged(ps + d + 0, o.x, tag);
            g_st_tagged(ps + d + 1, o.y, tag);
            g_st_tagged(ps + d + 2, o.z, tag);
            g_st_tagged(ps + d + 3, o.w, tag);
            if (d == 0) {
              g_st_tagged(ps + HD, ml[2 * h], tag);
              g_st_tagged(ps + HD + 1, ml[2 * h + 1], tag);
            }
          }
        }
      }
    }
    __syncthreads();  // LDS is reused by the next item
  }
  if (nsplit == 1) return;
  // 6. Merge, once all of this workgroup's own chunks are written (so it never
  //    waits on itself): the kvm * HD outputs of kv head g are split over
  //    MW = ceil(nsplit / kAttnMergeChunks) merging workgroups, those of chunks
  //    0, kAttnMergeChunks, 2 kAttnMergeChunks, ... (one per head up to that
  //    many chunks, where a single merger is fastest; at long contexts the
  //    reads a merger makes would otherwise be bound by one CU's read rate).
  //    Merger m takes outputs [m E / MW, (m + 1) E / MW).  T adjacent lanes
  //    share an output; each polls the
  //    (o, m, l) of every T-th chunk, eight per round trip, merges them online,
  //    and the T partials are combined by lane exchanges:
  //    M = max(M1, M2), L = L1 e^(M1 - M) + L2 e^(M2 - M), likewise O; the
  //    output is O / L.
  auto merge2 = [](float& M, float& L, float& O, float m2, float l2, float o2) {
    const float Mn = fmaxf(M, m2);
    if (Mn == -INFINITY) return;  // neither side holds a chunk yet
    const float c1 = M == -INFINITY ? 0.f : expf(M - Mn);
    const float c2 = m2 == -INFINITY ? 0.f : expf(m2 - Mn);
    L = L * c1 + l2 * c2;
    O = O * c1 + o2 * c2;
    M = Mn;
  };
  const int E = kvm * HD;
  const int R = nsplit <= kAttnMergeChunks       ? kAttnMergeChunks
                : nsplit <= 2 * kAttnMergeChunks ? a.merge_chunks_mid
                                                 : a.merge_chunks;
  const int MW = (nsplit + R - 1) / R;
  for (int it = blockIdx.x; it < items; it += gridDim.x) {
    const int g = it / nsplit;
    const int s = it - g * nsplit;
    if (s % R != 0) continue;
    const int mi = s / R;
    const int lo = static_cast<int>(static_cast<long long>(mi) * E / MW);
    const int cnt = static_cast<int>(static_cast<long long>(mi + 1) * E / MW) - lo;
    if (cnt <= 0) continue;
    // Lanes per output (uniform): one while a lane's eight-chunk round trip covers
    // every chunk, more at long contexts.
    int T = kWave;
    while (T > 1 && T * cnt > kPThreads) T >>= 1;
    if (nsplit <= 8) T = 1;
    const tagged_t* pg = a.attn_part + static_cast<size_t>(g) * a.attn_G * kvm * (HD + 2);
    tagged_t* outg = a.att + static_cast<size_t>(g) * kvm * HD;
    for (int base = tid; base < ((cnt * T + kWave - 1) / kWave) * kWave; base += kPThreads) {
      const int j = base / T, c = base - j * T;
      const bool active = j < cnt;
      const int idx = lo + (active ? j : 0);
      const int h = idx / HD, d = idx - h * HD;
      float M = -INFINITY, L = 0.f, O = 0.f;
      for (int k0 = c; k0 < nsplit && active; k0 += 8 * T) {
        // e < 8: o of chunk k0 + (e & 7) T; 8 <= e < 16: its m; 16 <= e < 24: its l.
        auto addr = [&](int e) {
          const int k = k0 + (e & 7) * T, kk = k < nsplit ? k : 0;
          const tagged_t* ps = pg + (static_cast<size_t>(kk) * kvm + h) * (HD + 2);
          return e < 8 ? ps + d : ps + HD + (e >> 4);
        };
        tagged_t v[24];
        unsigned int valid = 0;
#pragma unroll
        for (int e = 0; e < 24; ++e) {
          const bool ok = k0 + (e & 7) * T < nsplit;
          if (ok) valid |= 1u << e;
          v[e] = ok ? g_ld64(addr(e)) : 0;  // only the chunks that exist are read
        }
        poll_many<24>(a, tag, addr, valid, v);
#pragma unroll
        // A lane's first chunk has a finite max, so its own updates need no
        // guard (e^(-inf) = 0 clears the empty start).
        for (int k = 0; k < 8; ++k) {
          if (k0 + k * T < nsplit) {
            const float ms = val_of(v[8 + k]);
            const float Mn = fmaxf(M, ms);
            const float cm = expf(M - Mn), w = expf(ms - Mn);
            L = L * cm + val_of(v[16 + k]) * w;
            O = O * cm + val_of(v[k]) * w;
            M = Mn;
          }
        }
      }
      // Combine the T lanes of this output (adjacent lanes, T divides 64).
      for (int w = 1; w < T; w <<= 1)
        merge2(M, L, O, __shfl_xor(M, w), __shfl_xor(L, w), __shfl_xor(O, w));
      if (active && c == 0) g_st_tagged(outg + idx, O / L, tag);
    }
  }
}

// ---------------------------------------------------------------------------
// Short-context attention (pos + 1 <= attn_short_max).  Same semantics as
// attn_p_phase, but one item per query head covers every position, so no
// partials cross workgroups and there is no merge hand-off.  A thread owns
// one float4 (dims 4 sub .. 4 sub + 3) of one K/V row per pass: TPR = HD / 4
// lanes per row, RPP rows per pass, up to kAttnShortPasses passes, the K and
// V rows in registers.  q, the new K and V rows are polled straight into the
// same lanes (every row group holds a copy), so the Qwen3 q/k RMSNorm is a
// TPR-lane DPP sum and RoPE's rotate-half partner is the lane TPR / 2 away.
// Each wave reduces its rows to (m, l, o[HD]); one barrier, then HD / 4
// threads merge the eight waves and store the head's output.
// ---------------------------------------------------------------------------
constexpr int kAttnShortPasses = 8;
__host__ __device__ constexpr int attn_short_rows(int hd) {
  return kAttnShortPasses * (kPThreads / (hd / 4));
}
// LDS floats: per-wave partials [kPWaves][HD + 2], then per-wave inputs
// [kPWaves][7 HD] (q, new K, new V, cos, sin, qn, kn).
__host__ __device__ constexpr size_t attn_short_wp_floats(int hd) {
  return (static_cast<size_t>(kPWaves) * (hd + 2) + 3) & ~size_t(3);
}
__host__ __device__ constexpr size_t attn_short_lds_floats(int hd) {
  return attn_short_wp_floats(hd) + static_cast<size_t>(kPWaves) * 7 * hd;
}

// Sum over the W aligned lanes of a row group, in every lane of the group
// (bitwise equal in all of them: each step adds two values that are equal up
// to the order of the operands).
template <int W>
__device__ __forceinline__ float rowgroup_sum(float v) {
  if constexpr (W <= 16) {
    return group_sum_dpp<W>(v);
  } else {
    v = group_sum_dpp<16>(v);
    v += __shfl_xor(v, 16);
    if constexpr (W == 64) v += __shfl_xor(v, 32);
    return v;
  }
}
// Sum over the row groups of a wave (lanes W apart), in every lane.
template <int W>
__device__ __forceinline__ float across_groups_sum(float v) {
#pragma unroll
  for (int off = W; off < kWave; off <<= 1) v += __shfl_xor(v, off);
  return v;
}

// Raw buffer load of 16 bytes at byte offset `off` of a buffer of `bytes`
// bytes: offsets past the end return zeros and read no memory.
__device__ __forceinline__ f4 buf_ld4(__amdgpu_buffer_rsrc_t r, unsigned int off) {
  return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const float* base, unsigned int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), static_cast<short>(0), bytes,
                                           0x00020000);
}

template <int HD>
__device__ __forceinline__ void attn_short_phase(const PArgs& a, int layer, int pos,
                                                 unsigned int tag, float* lds, int trace_slot) {
  constexpr int TPR = HD / 4;
  constexpr int RPP = kPThreads / TPR;
  constexpr int NPM = kAttnShortPasses;
  constexpr int NE = (3 * HD + kWave - 1) / kWave;  // polled elements per lane
  constexpr int NT = (HD + kWave - 1) / kWave;      // table entries per lane and vector
  float* kcache = a.kc0 + layer * a.kv_layer;
  const float* vcache = a.vc0 + layer * a.kv_layer;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int sub = tid % TPR;
  const int rg = tid / TPR;
  const int kvm = a.kv_mul;
  const int n = pos + 1;
  const int items = a.KVH * kvm;
  const int ppos = pos / RPP, rgpos = pos - ppos * RPP;  // pass and row group of row pos
  float* wp = lds;  // [kPWaves][HD + 2]: per wave o[HD], m, l
  // Per wave: q, new K, new V [3 HD], then cos, sin, qn, kn [4 HD].
  float* wv = lds + attn_short_wp_floats(HD) + wave * 7 * HD;
  // The cached rows, through buffer loads bounded to rows < pos (row pos
  // comes from the QKV phase): rows past the context return zeros and cost
  // no memory traffic, so the code stays straight-line (exact wait counts)
  // and moves only the context's bytes.
  const unsigned int ctx_bytes = static_cast<unsigned int>(pos) * a.Dkv * 4;
  for (int it = blockIdx.x; it < items; it += gridDim.x) {
    // Items of one kv head sit KVH apart in workgroup order, on the same XCD
    // when KVH is a multiple of 8 (round-robin dispatch), sharing its L2.
    const int g = it % a.KVH, j = it / a.KVH;
    const int h = g * kvm + j;
    const size_t col = static_cast<size_t>(g) * HD + 4 * sub;

    // 1. Each wave polls q (head h) and the new K and V rows of kv head g
    //    once ([q | k | v], NE elements per lane); the first round is issued
    //    before the loads below, so that it is in flight while they are.
    tagged_t v[NE];
    auto addr = [&](int k) {
      int e = lane + k * kWave;
      e = e < 3 * HD ? e : 0;
      const tagged_t* base = e < HD       ? a.q + static_cast<size_t>(h) * HD
                             : e < 2 * HD ? a.knew + static_cast<size_t>(g) * HD - HD
                                          : a.vnew + static_cast<size_t>(g) * HD - 2 * HD;
      return base + e;
    };
    unsigned int valid = 0;
#pragma unroll
    for (int k = 0; k < NE; ++k) {
      v[k] = g_ld64(addr(k));
      if (lane + k * kWave < 3 * HD) valid |= 1u << k;
    }
    // 2. The position's RoPE table rows and the Qwen3 norm weights (NT per
    //    lane each), and the cached K and V rows.
    float tb[4][NT];
#pragma unroll
    for (int k = 0; k < NT; ++k) {
      const int d = lane + k * kWave < HD ? lane + k * kWave : 0;
      tb[0][k] = a.transform >= 1 ? g_rd(a.cos_t + static_cast<size_t>(pos) * HD + d) : 1.f;
      tb[1][k] = a.transform >= 1 ? g_rd(a.sin_t + static_cast<size_t>(pos) * HD + d) : 0.f;
      tb[2][k] = a.transform == 2 ? g_rd(a.qkn + static_cast<size_t>(layer) * 2 * HD + d) : 0.f;
      tb[3][k] = a.transform == 2 ? g_rd(a.qkn + static_cast<size_t>(layer) * 2 * HD + HD + d) : 0.f;
    }
    const __amdgpu_buffer_rsrc_t kb = buf_rsrc(kcache, ctx_bytes);
    const __amdgpu_buffer_rsrc_t vb = buf_rsrc(vcache, ctx_bytes);
    f4 kr[NPM], vr[NPM];
#pragma unroll
    for (int p = 0; p < NPM; ++p) {
      const unsigned int off = static_cast<unsigned int>((p * RPP + rg) * a.Dkv + col) * 4;
      kr[p] = buf_ld4(kb, off);
      vr[p] = buf_ld4(vb, off);
    }
    poll_many<NE>(a, tag, addr, valid, v);
    if (it == static_cast<int>(blockIdx.x)) trace_mark(a, trace_slot);  // inputs arrived
    // Through the wave's own LDS slice (in order within a wave: no barrier).
#pragma unroll
    for (int k = 0; k < NE; ++k)
      if (lane + k * kWave < 3 * HD) wv[lane + k * kWave] = val_of(v[k]);
#pragma unroll
    for (int k = 0; k < NT; ++k)
      if (lane + k * kWave < HD)
#pragma unroll
        for (int x = 0; x < 4; ++x) wv[3 * HD + x * HD + lane + k * kWave] = tb[x][k];
    f4 q4 = reinterpret_cast<const f4*>(wv)[sub];
    f4 k4 = reinterpret_cast<const f4*>(wv + HD)[sub];
    const f4 v4 = reinterpret_cast<const f4*>(wv + 2 * HD)[sub];
    const float* cs = wv + 3 * HD;
    const float* sn = wv + 4 * HD;

    // 3. Qwen3 per-head q/k RMSNorm (model/qwen3.cpp:485-500), then RoPE:
    //    interleaved pairs (2j, 2j + 1) and rotate-half pairs (j, j + HD / 2)
    //    both take table entry 2j (kernels/cpu/rope_kernel.cpp).
    if (a.transform == 2) {
      const f4 qn = reinterpret_cast<const f4*>(wv + 5 * HD)[sub];
      const f4 kn = reinterpret_cast<const f4*>(wv + 6 * HD)[sub];
      const float rq = 1.f / sqrtf(rowgroup_sum<TPR>(hsum(q4 * q4)) / static_cast<float>(HD) + a.qk_eps);
      const float rk = 1.f / sqrtf(rowgroup_sum<TPR>(hsum(k4 * k4)) / static_cast<float>(HD) + a.qk_eps);
      q4 = (rq * q4) * qn;
      k4 = (rk * k4) * kn;
    }
    if (a.transform >= 1) {
      if (a.rope_style == 0) {
#pragma unroll
        for (int k = 0; k < 4; k += 2) {
          const float c = cs[4 * sub + k], sv = sn[4 * sub + k];
          float a0 = q4[k], a1 = q4[k + 1];
          rope_pair(a0, a1, c, sv);
          q4[k] = a0;
          q4[k + 1] = a1;
          float b0 = k4[k], b1 = k4[k + 1];
          rope_pair(b0, b1, c, sv);
          k4[k] = b0;
          k4[k + 1] = b1;
        }
      } else {
        // Dims d < HD / 2 pair with d + HD / 2, held TPR / 2 lanes away.
        const bool lo = sub < TPR / 2;
        f4 qo, ko;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          qo[k] = __shfl_xor(q4[k], TPR / 2);
          ko[k] = __shfl_xor(k4[k], TPR / 2);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int ti = 2 * ((4 * sub + k) % (HD / 2));
          const float c = cs[ti], sv = sn[ti];
          float a0 = lo ? q4[k] : qo[k], a1 = lo ? qo[k] : q4[k];
          rope_pair(a0, a1, c, sv);
          q4[k] = lo ? a0 : a1;
          float b0 = lo ? k4[k] : ko[k], b1 = lo ? ko[k] : k4[k];
          rope_pair(b0, b1, c, sv);
          k4[k] = lo ? b0 : b1;
        }
      }
    }
    // Row pos joins the registers; its K row (transformed) goes to the cache.
#pragma unroll
    for (int p = 0; p < NPM; ++p) {
      const bool own = p == ppos && rg == rgpos;
      kr[p] = own ? k4 : kr[p];
      vr[p] = own ? v4 : vr[p];
    }
    if (j == 0 && rg == rgpos) *reinterpret_cast<f4*>(kcache + static_cast<size_t>(pos) * a.Dkv + col) = k4;

    // 4. Scores of this thread's rows (-inf past the context), the wave's
    //    maximum, its softmax sum and o = sum_t e_t V_t over its rows.
    float sc[NPM];
    float m = -INFINITY;
#pragma unroll
    for (int p = 0; p < NPM; ++p) {
      const float d = rowgroup_sum<TPR>(hsum(kr[p] * q4));
      sc[p] = p * RPP + rg < n ? d * a.scale : -INFINITY;
      m = fmaxf(m, sc[p]);
    }
    m = wave_max_dpp(m);
    float l = 0.f;
    f4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < NPM; ++p) {
      const float e = p * RPP + rg < n ? expf(sc[p] - m) : 0.f;  // a wave past the context: m = -inf
      l += e;
      o += e * vr[p];
    }
    l = across_groups_sum<TPR>(l);
    o.x = across_groups_sum<TPR>(o.x);
    o.y = across_groups_sum<TPR>(o.y);
    o.z = across_groups_sum<TPR>(o.z);
    o.w = across_groups_sum<TPR>(o.w);
    float* w = wp + wave * (HD + 2);
    if (lane < TPR) reinterpret_cast<f4*>(w)[sub] = o;
    if (lane == 0) {
      w[HD] = m;
      w[HD + 1] = l;
    }
    __syncthreads();
    // 5. Merge the waves: M = max m_w, L = sum l_w e^(m_w - M), O likewise
    //    (a wave without rows has m = -inf, weight 0); the output is O / L.
    if (tid < TPR) {
      float mw[kPWaves], lw[kPWaves];
      f4 ow[kPWaves];
#pragma unroll
      for (int x = 0; x < kPWaves; ++x) {
        mw[x] = wp[x * (HD + 2) + HD];
        lw[x] = wp[x * (HD + 2) + HD + 1];
        ow[x] = reinterpret_cast<const f4*>(wp + x * (HD + 2))[tid];
      }
      float M = mw[0];
#pragma unroll
      for (int x = 1; x < kPWaves; ++x) M = fmaxf(M, mw[x]);
      float L = 0.f;
      f4 O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int x = 0; x < kPWaves; ++x) {
        const float c = expf(mw[x] - M);
        L += lw[x] * c;
        O += c * ow[x];
      }
      tagged_t* op = a.att + static_cast<size_t>(h) * HD + 4 * tid;
      g_st_tagged(op + 0, O.x / L, tag);
      g_st_tagged(op + 1, O.y / L, tag);
      g_st_tagged(op + 2, O.z / L, tag);
      g_st_tagged(op + 3, O.w / L, tag);
    }
    __syncthreads();  // LDS is reused by the next item
  }
}

// ---------------------------------------------------------------------------
// Epilogues of the QKV, residual and SwiGLU phases.  `xres` holds this
// workgroup's rows of the residual stream (the WO and W2 phases split the D
// rows identically); `rn` is the RMSNorm scale of the phase's input.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void p_epilogue(PGp p, const PGeom& g, const float* red, int pos,
                                           unsigned int tag, float* xres, float rn) {
  const int ks = p->ks;
  const int epi = p->epi;
  if (epi == kEpiQkv) {
    for (int lr = threadIdx.x; lr < g.nloc; lr += kPThreads) {
      int sub, row;
      p_row(p, g, lr, sub, row);
      float v = rn * p_row_total(ks, red, lr);
      const float* b = p->bias[sub];
      if (b) v = v + g_rd(b + row);
      g_st_tagged(p->out[sub] + row, v, tag);
      if (sub == 2) p->vcache[static_cast<size_t>(pos) * p->rows[2] + row] = v;
    }
  } else if (epi == kEpiResid) {
    tagged_t* out = p->out[0];
    for (int lr = threadIdx.x; lr < g.nloc; lr += kPThreads) {
      const float x = xres[lr] + p_row_total(ks, red, lr);
      xres[lr] = x;
      g_st_tagged(out + g.base + lr, x, tag);
    }
  } else if (epi == kEpiSwiglu) {
    tagged_t* out = p->out[0];
    for (int lr = threadIdx.x; lr < g.cnt; lr += kPThreads) {
      const float a1 = rn * p_row_total(ks, red, lr);
      const float a3 = rn * p_row_total(ks, red, lr + g.cnt);
      // kernels/cpu/swiglu_kernel.cpp:21-22
      const float s = a1 * (1.0f / (1.0f + expf(-a1)));
      g_st_tagged(out + g.base + lr, s * a3, tag);
    }
  }
}

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
// SHORT selects the attention path at compile time (short-context items, or
// the chunked split with merges): a kernel holding both needs more registers
// than a wave has.  The host launches the variant that fits the position.
template <bool Q8, int NB, int HD, bool SHORT>
__global__ __launch_bounds__(kPThreads) void k_decode_persistent(PArgs a) {
  extern __shared__ __align__(16) float lds[];
  __shared__ float sred[2 * kPWaves];
  __shared__ int s_last;
  __shared__ int s_claim;
  __shared__ float s_bv[kPWaves];
  __shared__ int s_bi[kPWaves];
  const PStepState st = *a.st;  // written by the previous launch
  const int pos = st.pos;
  const int token = st.token;
  if (pos < 0 || pos >= a.S || token < 0 || token >= a.V) {
    if (blockIdx.x == 0 && threadIdx.x == 0) g_st(a.err, kDevErrPos);
    return;
  }
  if ((pos + 1 <= a.attn_short_max) != SHORT) {
    if (blockIdx.x == 0 && threadIdx.x == 0) g_st(a.err, kDevErrVariant);
    return;
  }
  const bool sample = pos + 1 >= st.prompt_len;
  const unsigned int epoch = g_rd(a.epoch);
  const float* emb_row = a.emb + static_cast<size_t>(token) * a.D;
  const PGp ph = (PGp)(a.ph);
  const int ncls = 4 * a.L;  // index of the classifier phase
  float* xs = lds;
  float* red = lds + a.red_off;
  float* xres = lds + a.xres_off;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int slot = 0;
  // RoPE table entries of this launch's position (every pair a thread
  // rotates has j = tid % (HD / 2)).
  float rope_c = 1.f, rope_s = 0.f;
  if (a.transform >= 1) {
    const int j = threadIdx.x % (HD / 2);
    rope_c = g_rd(a.cos_t + static_cast<size_t>(pos) * HD + 2 * j);
    rope_s = g_rd(a.sin_t + static_cast<size_t>(pos) * HD + 2 * j);
  }
  constexpr bool attn_short = SHORT;
  if (a.trace) {
    for (int s = threadIdx.x; s < a.trace_slots; s += kPThreads) trace_lds(a)[s] = 0;
    __syncthreads();
  }
  trace_mark(a, slot++);

  {
    // This workgroup's rows of the residual stream start as the embedding row.
    const PGeom gr = p_geom(ph + 1);
    for (int lr = threadIdx.x; lr < gr.nloc; lr += kPThreads) xres[lr] = g_rd(emb_row + gr.base + lr);
  }
  float bv = -INFINITY;
  int bi = INT_MAX;
  for (int k = 0; k <= ncls; ++k) {
    const PGp p = ph + k;
    const bool is_cls = k == ncls;
    // The next GEMV phase (none after the last layer of a prompt position).
    const PGp pn = k + 1 < ncls ? ph + k + 1 : (k + 1 == ncls && sample ? ph + ncls : nullptr);
    const PGeom g = p_geom(p);
    const unsigned int tag_in = epoch * kTagLayers + p->in_layer + 1;
    const unsigned int tag = epoch * kTagLayers + p->layer + 1;
    // The phase's first weight segment is requested before its input is
    // polled, so that the weights are on their way during the hand-off.
    PChunk<Q8> A[NB];
    {
      PCur c0{0, 0, 0};
      p_seg_issue<Q8, NB>(p, g, c0, A);
    }
    stage_vec<Q8>(a, p->in, tag_in, emb_row, p->norm, p->cols, xs, sred);
    trace_mark(a, slot++);
    // Classifier: claim the first dynamic block now; the answer is needed
    // only after the static rows.
    unsigned int cls_claim = 0;
    if (is_cls && p->dyn > 0 && threadIdx.x == 0) cls_claim = g_arrive(a.cls_next);
    p_stream<Q8, NB>(p, g, A, xs, red);
    // RMSNorm scale of this phase's input (1 without a norm).
    const float rn = p->norm ? norm_scale(sred, p->cols, a.eps) : 1.f;
    if (is_cls) {
      // Logits (plain stores, read by the host after the launch) and this
      // workgroup's (max, first index) pair (sampler/argmax_sampler.cpp:5-13).
      float* logits = p->logits;
      const int ks = p->ks;
      // The dynamic rows: blocks claimed one ahead (the claim is in flight
      // while a block streams), each block's first segment requested before
      // the previous block's rows are read out of LDS.
      const int nblk = p->dyn > 0 ? (p->dyn + p->blk - 1) / p->blk : 0;
      int blk = nblk;
      PGeom gd = g;
      PChunk<Q8> D[NB];
      if (nblk > 0) {
        if (threadIdx.x == 0) s_claim = static_cast<int>(cls_claim);
        __syncthreads();
        blk = s_claim;
        if (blk < nblk) {
          gd = p_geom_block(p, blk);
          PCur c0{0, 0, 0};
          p_seg_issue<Q8, NB>(p, gd, c0, D);
        }
      }
      for (int lr = threadIdx.x; lr < g.nloc; lr += kPThreads) {
        const float v = rn * p_row_total(ks, red, lr);
        logits[g.base + lr] = v;
        argmax_merge(bv, bi, v, g.base + lr);
      }
      while (blk < nblk) {
        unsigned int claim = 0;
        if (threadIdx.x == 0) claim = g_arrive(a.cls_next);
        __syncthreads();  // the previous rows are read out of red
        p_stream<Q8, NB>(p, gd, D, xs, red);
        if (threadIdx.x == 0) s_claim = static_cast<int>(claim);
        __syncthreads();
        const int nxt = s_claim;
        const PGeom gc = gd;
        if (nxt < nblk) {
          gd = p_geom_block(p, nxt);
          PCur c0{0, 0, 0};
          p_seg_issue<Q8, NB>(p, gd, c0, D);
        }
        for (int lr = threadIdx.x; lr < gc.nloc; lr += kPThreads) {
          const float v = rn * p_row_total(ks, red, lr);
          logits[gc.base + lr] = v;
          argmax_merge(bv, bi, v, gc.base + lr);
        }
        blk = nxt;
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
        g_st(a.am_pi + blockIdx.x, bi);
      }
      trace_mark(a, slot++);
      break;
    }
    p_epilogue(p, g, red, pos, tag, xres, rn);
    __syncthreads();  // red and xres are rewritten by the next phase
    trace_mark(a, slot++);
    if (!pn) break;  // last layer of a prompt position: no classifier
    if ((k & 3) == 0) {  // after QKV: attention of layer k / 4
      const int items = attn_short ? a.KVH * a.kv_mul
                                   : a.KVH * ((pos + attn_chunk(HD)) / attn_chunk(HD));
      const int b = static_cast<int>(blockIdx.x);
      if (b >= items) {
        trace_mark(a, slot);  // no attention item: "inputs arrived" = now
        // Idle until the attention output arrives: pull this workgroup's
        // W1/W3 rows into L2, and slices of the W1/W3 rows of the attention
        // workgroups of the same XCD (under round-robin dispatch), which have
        // no time to.
        const int nw = static_cast<int>(gridDim.x);
        // The attention phase, and so the window for the pull, lengthens with
        // the number of attention items: pull up to 1.5x as much then.
        const int rows = attn_short ? a.short_touch_rows
                                    : a.w13_touch_rows + a.w13_touch_rows * min(items, nw / 2) / nw;
        if (rows > 0) {
          if (a.touch_delay > 0) {
            const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
            while (__builtin_amdgcn_s_memrealtime() - t0 < static_cast<unsigned long long>(a.touch_delay))
              __builtin_amdgcn_s_sleep(4);
          }
          // The attention workgroups of this XCD (x, x + 8, ... below items,
          // under round-robin dispatch) cannot pull their own rows: the other
          // workgroups of the XCD share that work, an even slice each (at
          // most two attention workgroups' rows per slice are pulled).
          const PGp pw = pn + 1;  // W1/W3
          const int x = b & 7;
          const int cx = items > x ? (items - x + 7) / 8 : 0;  // attention workgroups
          const int h = (b - x) / 8 - cx, nh = (nw - x + 7) / 8 - cx;
          const long long tot = static_cast<long long>(cx) * rows;
          const int q0 = static_cast<int>(tot * h / nh), q1 = static_cast<int>(tot * (h + 1) / nh);
          const int j0 = q0 / rows, j1 = j0 + 1;
          TouchSpan s[6];
          p_touch_rows<Q8>(pw, b, 0, rows, s[0], s[1]);
          p_touch_rows<Q8>(pw, x + 8 * j0, q0 - j0 * rows, min(q1 - j0 * rows, rows), s[2], s[3]);
          p_touch_rows<Q8>(pw, x + 8 * min(j1, max(cx - 1, 0)), 0,
                           j1 < cx ? min(q1 - j1 * rows, rows) : 0, s[4], s[5]);
          const unsigned int t = p_touch_lines(s[0], s[1], s[2], s[3], s[4], s[5]);
          asm volatile("" ::"v"(t));  // keeps the loads
        }
      }
      if constexpr (SHORT)
        attn_short_phase<HD>(a, k >> 2, pos, tag, lds, slot);
      else
        attn_p_phase<HD>(a, a.at + (k >> 2), pos, tag, lds, slot, rope_c, rope_s);
      ++slot;
      trace_mark(a, slot++);
    }
  }

  if (a.trace) {
    __syncthreads();
    for (int s = threadIdx.x; s < a.trace_slots; s += kPThreads)
      a.trace[static_cast<size_t>(s) * gridDim.x + blockIdx.x] = trace_lds(a)[s];
  }

  // End of step: the last workgroup to arrive samples (or takes the next
  // prompt token) and advances the device state for the next launch.
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
      argmax_merge(bv, bi, g_ld(a.am_pv + b), g_ld(a.am_pi + b));
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
  const bool wrap = epoch + 1 >= kEpochWrap;
  if (wrap) {
    for (long long i = threadIdx.x; i < a.attn_part_n; i += kPThreads) a.attn_part[i] = 0;
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
    *a.epoch = wrap ? 0u : epoch + 1;
    // Every workgroup has arrived, so every claim is made (each workgroup's
    // last claim was past the blocks).
    g_st(a.cls_next, 0u);
    g_st(a.am_cnt, 0u);
  }
}

}  // namespace kl
