// Fused batch-1 decode engine for the Llama2 / Llama3 / Qwen2 / Qwen3 step of
// the reference (model/llama3.cpp:146-166, :599-744; model/qwen2.cpp:205-225,
// :640-801; model/qwen3.cpp:147-167, :459-640).
//
// One token step is 5 kernels per layer plus 2 per token, replayed as a HIP
// graph:
//   embed      x = E[token]                       (state.token, device resident)
//   per layer
//     qkv      RMSNorm(x) staged in LDS, [Wq;Wk;Wv] GEMV, + bias (Qwen2),
//              q -> q buffer, k/v -> cache slot at state.pos
//     attn     (q/k norm) + RoPE + split-K attention + cross-chunk merge
//     wo       x += Wo . attn
//     w13      RMSNorm(x) staged in LDS, W1 and W3 rows side by side,
//              h = silu(W1 x) * (W3 x)
//     w2       x += W2 . h
//   cls        final RMSNorm staged in LDS, classifier GEMV, logits, argmax
//              partials, last workgroup picks the token and advances state
// Every kernel reads the position from device memory, so the captured graph
// is position independent; between replays only the device state changes.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "attn.hpp"
#include "device.hpp"
#include "gemm_run.hpp"
#include "gemv.hpp"
#include "kuiper_hip.h"
#include "persist.hpp"

using namespace kl;

namespace {

typedef PStepState StepState;
constexpr int kMaxPwgPerCu = 4;  // persistent workgroups per CU (KL_PWG_PER_CU)

inline int rc(hipError_t e) { return e == hipSuccess ? KL_OK : static_cast<int>(e); }

// ---------------------------------------------------------------------------
// Kernels.  Each GEMV-shaped kernel is run_tiles() with its own row map,
// input staging and epilogue (see gemv.hpp); blockDim = 64 * KS * G.
// ---------------------------------------------------------------------------
constexpr int kRedFloats = 32;

// [Wq; Wk; Wv] . RMSNorm(x); q -> q buffer, k/v -> cache slot at state.pos,
// + bias (Qwen2).  Layer 0 reads its input straight from the embedding row of
// state.token and workgroup 0 stores it as the residual stream x.
struct QkvArgs {
  const float* x;
  const float* emb;  // layer 0 only: embedding table
  float* x_out;      // layer 0 only: residual stream
  const StepState* st;
  const float* nw;
  float eps;
  int D, Dq, Dkv;
  ColGeom g;
  WView wq, wk, wv;
  const float *bq, *bk, *bv;
  float* q_out;
  float* kcache;  // layer base
  float* vcache;  // layer base
};

template <bool Q8, int U>
__global__ __launch_bounds__(512) void k_qkv(QkvArgs a) {
  extern __shared__ float xs[];
  __shared__ float red[kRedFloats];
  const int pos = a.st->pos;
  const int total = a.Dq + 2 * a.Dkv;
  auto rows = [&](int u, int, WView& m, size_t& row) {
    if (u < a.Dq) {
      m = a.wq;
      row = u;
    } else if (u < a.Dq + a.Dkv) {
      m = a.wk;
      row = u - a.Dq;
    } else {
      m = a.wv;
      row = u - a.Dq - a.Dkv;
    }
  };
  auto stage = [&]() {
    const float* x = a.emb ? a.emb + static_cast<size_t>(a.st->token) * a.D : a.x;
    if (a.emb && blockIdx.x == 0)
      for (int i = threadIdx.x; i < a.D; i += blockDim.x) a.x_out[i] = x[i];
    stage_input(x, a.nw, a.eps, a.D, xs, red);
  };
  auto epi = [&](int u, const float (&v)[1]) {
    if ((threadIdx.x & 63) != 0) return;
    if (u < a.Dq) {
      a.q_out[u] = a.bq ? v[0] + a.bq[u] : v[0];
    } else if (u < a.Dq + a.Dkv) {
      const int r = u - a.Dq;
      a.kcache[static_cast<size_t>(pos) * a.Dkv + r] = a.bk ? v[0] + a.bk[r] : v[0];
    } else {
      const int r = u - a.Dq - a.Dkv;
      a.vcache[static_cast<size_t>(pos) * a.Dkv + r] = a.bv ? v[0] + a.bv[r] : v[0];
    }
  };
  run_tiles<Q8, 1, U>(a.g, total, xs, red, rows, stage, epi);
}

// x[row] += W[row, :] . in   (output projection and down projection + residual)
struct ResArgs {
  const float* in;
  int rows;
  ColGeom g;
  WView w;
  float* x;
};

template <bool Q8, int U>
__global__ __launch_bounds__(512) void k_gemv_residual(ResArgs a) {
  extern __shared__ float xs[];
  __shared__ float red[kRedFloats];
  auto rows = [&](int u, int, WView& m, size_t& row) {
    m = a.w;
    row = u;
  };
  auto stage = [&]() { stage_input(a.in, nullptr, 0.f, a.g.cols, xs, red); };
  auto epi = [&](int u, const float (&v)[1]) {
    if ((threadIdx.x & 63) == 0) a.x[u] = a.x[u] + v[0];
  };
  run_tiles<Q8, 1, U>(a.g, a.rows, xs, red, rows, stage, epi);
}

// h[r] = silu(W1[r] . xn) * (W3[r] . xn), xn = RMSNorm(x): a tile is row r of
// W1 and row r of W3 (R = 2).
struct W13Args {
  const float* x;
  const float* nw;
  float eps;
  int D, F;
  ColGeom g;
  WView w1, w3;
  float* h;
};

template <bool Q8, int U>
__global__ __launch_bounds__(512) void k_w13_swiglu(W13Args a) {
  extern __shared__ float xs[];
  __shared__ float red[kRedFloats];
  auto rows = [&](int u, int r, WView& m, size_t& row) {
    m = r == 0 ? a.w1 : a.w3;
    row = u;
  };
  auto stage = [&]() { stage_input(a.x, a.nw, a.eps, a.D, xs, red); };
  auto epi = [&](int u, const float (&v)[2]) {
    if ((threadIdx.x & 63) != 0) return;
    // kernels/cpu/swiglu_kernel.cpp:21-22
    const float s = v[0] * (1.0f / (1.0f + expf(-v[0])));
    a.h[u] = s * v[1];
  };
  run_tiles<Q8, 2, U>(a.g, a.F, xs, red, rows, stage, epi);
}

// Classifier + greedy sampling.
struct ClsArgs {
  const float* x;
  const float* nw;
  float eps;
  int D, V;
  ColGeom g;
  WView w;
  float* logits;
  float* pv;
  int* pi;
  unsigned int* counter;
  StepState* st;
  const int32_t* prompt;
  int32_t* out_tokens;
};

template <bool Q8, int U>
__global__ __launch_bounds__(512) void k_cls_argmax(ClsArgs a) {
  extern __shared__ float xs[];
  __shared__ float red[kRedFloats];
  __shared__ float sv[16];
  __shared__ int si[16];
  __shared__ int s_last;
  const int pos = a.st->pos;
  const int P = a.st->prompt_len;
  if (pos + 1 < P) {
    // A prompt position whose successor is already known: the reference
    // computes logits here and discards them (demo/main.cpp:20-22, is_prompt);
    // only the device state advances.
    if (blockIdx.x == 0 && threadIdx.x == 0) {
      a.st->token = a.prompt[pos + 1];
      a.st->pos = pos + 1;
    }
    return;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  float bv = -INFINITY;
  int bi = INT_MAX;
  auto rows = [&](int u, int, WView& m, size_t& row) {
    m = a.w;
    row = u;
  };
  auto stage = [&]() { stage_input(a.x, a.nw, a.eps, a.D, xs, red); };
  auto epi = [&](int u, const float (&v)[1]) {
    if (lane == 0) a.logits[u] = v[0];
    argmax_merge(bv, bi, v[0], u);
  };
  run_tiles<Q8, 1, U>(a.g, a.V, xs, red, rows, stage, epi);
  // Every lane of a wave holds the same (bv, bi); merge the waves.
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < nw; ++w) argmax_merge(bv, bi, sv[w], si[w]);
    store_coherent(a.pv + blockIdx.x, bv);
    store_coherent(a.pi + blockIdx.x, bi);
    wait_mem();
    const unsigned int prev = arrive(a.counter);
    s_last = prev == gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last) return;
  bv = -INFINITY;
  bi = INT_MAX;
  for (int b = threadIdx.x; b < static_cast<int>(gridDim.x); b += blockDim.x)
    argmax_merge(bv, bi, load_coherent(a.pv + b), load_coherent(a.pi + b));
  wave_argmax(bv, bi);
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < nw; ++w) argmax_merge(bv, bi, sv[w], si[w]);
    a.st->sampled = bi;
    a.st->token = bi;
    a.out_tokens[pos] = bi;
    a.st->pos = pos + 1;
    *a.counter = 0u;
  }
}

// ---------------------------------------------------------------------------
// Model image parsing (host).  Offsets follow model/model.cpp:41-141 and the
// loaders model/llama3.cpp:183-422 (fp32 / int8), model/qwen2.cpp:348-485
// (bias after each of wq/wk/wv) and model/qwen3.cpp:186-299.
// ---------------------------------------------------------------------------
struct HostTensor {
  const char* ptr = nullptr;
  size_t bytes = 0;
};

struct LayerHost {
  HostTensor rms_att, rms_ffn, wq, wk, wv, wo, w1, w2, w3, sq, sk, sv, so, s1, s2, s3, bq, bk, bv,
      qn, kn;
};

struct ImageLayout {
  int family = 0, quant = 0, gs = 0;
  int D = 0, Dq = 0, Dkv = 0, F = 0, L = 0, H = 0, KVH = 0, V = 0, S = 0, hd = 0;
  bool tied = false;
  HostTensor emb, rms_final, wcls, scls;
  std::vector<LayerHost> layers;
};

int parse_image(const void* image, size_t size, int family, int quant, ImageLayout* out) {
  if (!image || family < KL_FAMILY_LLAMA2 || family > KL_FAMILY_QWEN3) return KL_EINVAL;
  const bool qwen3 = family == KL_FAMILY_QWEN3;
  // int8 images: the Llama layout (llama3.cpp:183-287), also for Qwen2
  // (qwen2.cpp:242-346, no biases); Qwen3 has none.
  if (quant && qwen3) return KL_EUNSUPP;
  const size_t header_ints = (qwen3 || quant) ? 8 : 7;
  if (size < header_ints * 4) return KL_EFORMAT;
  const int32_t* h = static_cast<const int32_t*>(image);
  ImageLayout& m = *out;
  m.family = family;
  m.quant = quant;
  const int32_t dim = h[0], hidden = h[1], vocab = h[5];
  m.L = h[2];
  m.H = h[3];
  m.KVH = h[4];
  m.S = h[6];
  if (dim <= 0 || hidden <= 0 || m.L <= 0 || m.H <= 0 || m.KVH <= 0 || vocab == 0 || m.S <= 0 ||
      dim % m.H != 0 || m.H % m.KVH != 0)
    return KL_EFORMAT;
  m.V = std::abs(vocab);
  m.hd = dim / m.H;
  m.Dq = dim;
  m.Dkv = dim / m.H * m.KVH;
  if (qwen3) {
    m.D = hidden;
    m.F = h[7];
    m.tied = false;
    if (m.F <= 0) return KL_EFORMAT;
  } else {
    m.D = dim;
    m.F = hidden;
    m.tied = vocab > 0;
  }
  if (quant) {
    m.gs = h[7];
    if (m.gs <= 0) return KL_EFORMAT;
    if (m.tied) return KL_EUNSUPP;  // llama3.cpp:258-267 reads fp32 bytes as int8
  }
  const char* base = static_cast<const char*>(image) + header_ints * 4;
  const size_t avail = size - header_ints * 4;
  size_t off = 0;
  bool overflow = false;
  auto take = [&](size_t bytes) {
    HostTensor t{base + off, bytes};
    off += bytes;
    if (off > avail) overflow = true;
    return t;
  };
  auto f32 = [&](size_t n) { return take(n * 4); };
  const size_t L = m.L, D = m.D, Dq = m.Dq, Dkv = m.Dkv, F = m.F, V = m.V;
  m.layers.assign(L, LayerHost{});
  if (quant) {
    const size_t gs = m.gs;
    auto q8 = [&](size_t n, HostTensor* w, HostTensor* s) {
      if (n % gs != 0) overflow = true;
      *w = take(n);
      *s = f32(n / gs);
    };
    for (auto& l : m.layers) q8(Dq * D, &l.wq, &l.sq);
    for (auto& l : m.layers) q8(Dkv * D, &l.wk, &l.sk);
    for (auto& l : m.layers) q8(Dkv * D, &l.wv, &l.sv);
    for (auto& l : m.layers) q8(D * Dq, &l.wo, &l.so);
    for (auto& l : m.layers) q8(F * D, &l.w1, &l.s1);
    for (auto& l : m.layers) q8(D * F, &l.w2, &l.s2);
    for (auto& l : m.layers) q8(F * D, &l.w3, &l.s3);
    q8(V * D, &m.wcls, &m.scls);
    m.emb = f32(V * D);
    for (auto& l : m.layers) l.rms_att = f32(D);
    for (auto& l : m.layers) l.rms_ffn = f32(D);
    m.rms_final = f32(D);
  } else if (qwen3) {
    for (auto& l : m.layers) l.rms_att = f32(D);
    for (auto& l : m.layers) l.rms_ffn = f32(D);
    m.rms_final = f32(D);
    m.emb = f32(V * D);
    for (auto& l : m.layers) l.wq = f32(Dq * D);
    for (auto& l : m.layers) l.qn = f32(m.hd);
    for (auto& l : m.layers) l.wk = f32(Dkv * D);
    for (auto& l : m.layers) l.kn = f32(m.hd);
    for (auto& l : m.layers) l.wv = f32(Dkv * D);
    for (auto& l : m.layers) l.wo = f32(D * Dq);
    for (auto& l : m.layers) l.w1 = f32(F * D);
    for (auto& l : m.layers) l.w2 = f32(D * F);
    for (auto& l : m.layers) l.w3 = f32(F * D);
    m.wcls = f32(V * D);
  } else {
    const bool bias = family == KL_FAMILY_QWEN2;
    m.emb = f32(V * D);
    for (auto& l : m.layers) l.rms_att = f32(D);
    for (auto& l : m.layers) {
      l.wq = f32(Dq * D);
      if (bias) l.bq = f32(Dq);
    }
    for (auto& l : m.layers) {
      l.wk = f32(Dkv * D);
      if (bias) l.bk = f32(Dkv);
    }
    for (auto& l : m.layers) {
      l.wv = f32(Dkv * D);
      if (bias) l.bv = f32(Dkv);
    }
    for (auto& l : m.layers) l.wo = f32(D * Dq);
    for (auto& l : m.layers) l.rms_ffn = f32(D);
    for (auto& l : m.layers) l.w1 = f32(F * D);
    for (auto& l : m.layers) l.w2 = f32(D * F);
    for (auto& l : m.layers) l.w3 = f32(F * D);
    m.rms_final = f32(D);
    f32(static_cast<size_t>(m.S) * m.hd);  // freq_cos + freq_sin, unused
    if (!m.tied) m.wcls = f32(V * D);
  }
  if (overflow) return KL_EFORMAT;
  return KL_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Engine.
// ---------------------------------------------------------------------------
// bf16 planes (k_split3) of one layer's fp32 projections for the
// split-product prefill GEMM: 3 planes of N x K each.
struct XPlanes {
  const void *q, *k, *v, *o, *w1, *w2, *w3;
  // Bit i set: matrix i (q k v o w1 w2 w3) has all-zero planes 1 and 2 (bf16-exact
  // weights), so its GEMMs load plane 0 only and form three products.
  unsigned one;
};

struct LayerDev {
  const float *rms_att, *rms_ffn, *bq, *bk, *bv, *qn, *kn;
  WView wq, wk, wv, wo, w1, w2, w3;
  XPlanes xp;
};

struct kl_engine {
  ImageLayout lay;  // host pointers are not kept valid after create
  int family = 0, quant = 0, chunk_shift = 0;
  float eps = 1e-5f, theta = 1e4f;
  int rope_style = KL_ROPE_INTERLEAVED, transform = 1;
  int cus = 256;
  hipStream_t stream = nullptr;
  char* arena = nullptr;
  size_t arena_bytes = 0, weight_bytes = 0;
  const float* emb = nullptr;
  const float* rms_final = nullptr;
  WView wcls{};
  std::vector<LayerDev> layers;
  float *sin_t = nullptr, *cos_t = nullptr, *kcache = nullptr, *vcache = nullptr;
  float *x = nullptr, *q = nullptr, *att = nullptr, *h = nullptr, *logits = nullptr;
  float* attn_part = nullptr;
  unsigned int* attn_counters = nullptr;
  float* am_pv = nullptr;
  int* am_pi = nullptr;
  unsigned int* am_counter = nullptr;
  unsigned int* cls_next = nullptr;  // dynamic classifier blocks handed out (same 64-byte slot)
  StepState* st = nullptr;
  StepState* st_host = nullptr;  // pinned staging
  int32_t* prompt = nullptr;
  int32_t* out_tokens = nullptr;
  MhaPlan attn{};
  int grid_cap = 2048;
  struct GemvLaunch {
    ColGeom g;
    int U;
    dim3 grid, block;
    size_t lds;
  } l_qkv, l_wo, l_w13, l_w2, l_cls;
  bool use_graph = true;
  hipGraphExec_t graph_exec = nullptr;
  hipGraph_t graph = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  // Persistent step (persist.hpp): one launch per token.  The multi-kernel
  // step until setup_persistent() has shown that the persistent grid fits
  // (every early return there leaves this mode).
  int mode = KL_MODE_MULTI;
  bool persistent_ok = false;  // the persistent kernel fits this device and model
  // The persistent grid is launched with hipLaunchKernel where the occupancy
  // query shows every workgroup resident at once (one per CU), else with
  // hipLaunchCooperativeKernel.  The plain launch saves ~20 us per token and
  // the profiler's kernel trace survives it; every wait in the kernel is
  // bounded, so a grid that were not co-resident would end with the device
  // error flag set, not hang.  KL_PERSISTENT_LAUNCH=cooperative forces the
  // cooperative API.
  bool plain_launch = false;
  int nwg = 0;                 // workgroups (co-resident)
  size_t p_lds = 0;
  size_t p_lds_traced = 0;     // p_lds + the trace slots (traced launches)
  bool trace_ok = false;       // the traced launch is co-resident too
  const void* p_kernel = nullptr;        // long-context attention variant
  const void* p_kernel_short = nullptr;  // short-context attention variant
  int host_pos = 0;  // position of the next persistent launch (chooses the variant)
  PGemv* d_ph = nullptr;       // [4L + 1] phase descriptors (arena)
  // Row split per workgroup, weighted by measured streaming speed (empty:
  // balanced).  d_split holds 4 tables of nwg + 1 row offsets: QKV rows, D, F, V.
  std::vector<double> wg_weight;
  int* d_split = nullptr;
  PAttn* d_at = nullptr;       // [L]
  float* qkn = nullptr;        // [L][2][hd] Qwen3 q and k norm weights (arena)
  tagged_t *t_q = nullptr, *t_k = nullptr, *t_v = nullptr, *t_att = nullptr;  // tagged
  tagged_t *t_xb = nullptr, *t_h = nullptr, *t_x = nullptr;                    //   hand-off
  tagged_t* t_part = nullptr;  // attention split partials (tagged)
  unsigned int* epoch = nullptr;
  int* derr = nullptr;
  int* derr_host = nullptr;    // pinned
  PArgs pargs{};
  // Batched prompt prefill (kl_engine_prefill): scratch for one chunk of
  // rows, allocated on first use.
  bool use_prefill = false;
  // fp32 images: the projections run as split-product GEMMs (k_gemm_x6) on
  // bf16 planes of the weights (xw_buf, built on the first prefill, 1.5x the
  // fp32 projection bytes) and of each GEMM input (pf_ax).
  bool pf_x6 = false;
  // int8 images: chunks of at most 32 rows run k_gemm_q8s over the
  // projections prepacked into xw_buf (built on the first such prefill; the
  // int8 bytes plus the scales again), the GEMM inputs split into pf_ax.
  bool pf_q8s = false;
  char* xw_buf = nullptr;
  void* pf_ax = nullptr;        // planes of pf_rows x max(D, Dq, F) (x6_plane_bytes)
  int pf_rows = 0;              // rows the scratch holds
  char* pf_buf = nullptr;       // one allocation for everything below
  float *pf_x = nullptr, *pf_xn = nullptr, *pf_q = nullptr, *pf_att = nullptr;
  float *pf_h1 = nullptr, *pf_h3 = nullptr, *pf_xlast = nullptr;
  float* pf_ws = nullptr;       // split-K partials (prefill_scratch sizes them)
  size_t pf_ws_bytes = 0;
  void* pf_aws = nullptr;       // the attention's stream-K records
  size_t pf_aws_bytes = 0;
  int32_t* pf_tok = nullptr;    // [seq_len] prompt ids
  int32_t* pf_next = nullptr;
  void* pf_am = nullptr;        // argmax workspace (zeroed once)
  size_t pf_am_bytes = 0;
};

namespace {

// GEMV launch plan for `units` row units over `cols` columns: U = 4 chunks
// per lane per slice (4 KiB of a row per wave) with KS waves per row, or U = 8
// when a row would need more than kMaxKs slices; G rows per workgroup pass.
// Measured on MI355X (cold HBM): 4 KiB tiles with split-K and a grid of two
// workgroups per CU stream the 1 GB classifier at ~7 TB/s.
kl_engine::GemvLaunch plan_gemv(const kl_engine* e, int units, int cols) {
  kl_engine::GemvLaunch L;
  const bool q8 = e->quant != 0;
  const ColGeom g8 = make_geom(cols, q8, 8, e->lay.gs), g4 = make_geom(cols, q8, 4, e->lay.gs);
  const bool use4 = g4.ks <= kMaxKs;
  L.U = use4 ? 4 : 8;
  L.g = use4 ? g4 : g8;
  const int G = row_groups_for(L.g.ks);
  const int nblk = (units + G - 1) / G;
  L.grid = dim3(std::max(1, std::min(nblk, e->grid_cap)));
  L.block = dim3(kWave * L.g.ks * G);
  L.lds = static_cast<size_t>(cols) * sizeof(float);
  return L;
}

// Kernel kinds, in launch order within a layer; used by the profiler.
enum KernelKind { kKEmbed = 0, kKQkv, kKAttn, kKWo, kKW13, kKW2, kKCls, kKStep, kKinds, kKEnd };

// With `marks` set (eager profiling only), an event is recorded on the
// stream before every launch and after the last one; marks[i] then brackets
// kernel i and kinds[i] names it.
struct Marks {
  std::vector<hipEvent_t>* ev;
  std::vector<int>* kinds;
};

inline void mark(hipStream_t s, Marks* mk, int kind) {
  if (!mk) return;
  hipEvent_t ev;
  if (hipEventCreate(&ev) != hipSuccess) return;
  (void)hipEventRecord(ev, s);
  mk->ev->push_back(ev);
  mk->kinds->push_back(kind);
}

#define KL_GEMV_LAUNCH(KERNEL, Q8, L, S, ARGS)                                        \
  do {                                                                                \
    if ((L).U == 8)                                                                   \
      hipLaunchKernelGGL((KERNEL<Q8, 8>), (L).grid, (L).block, (L).lds, (S), (ARGS)); \
    else                                                                              \
      hipLaunchKernelGGL((KERNEL<Q8, 4>), (L).grid, (L).block, (L).lds, (S), (ARGS)); \
  } while (0)

template <bool Q8>
int launch_step_t(kl_engine* e, Marks* mk) {
  const ImageLayout& m = e->lay;
  hipStream_t s = e->stream;
  const size_t kv_layer = static_cast<size_t>(m.S) * m.Dkv;
  for (int l = 0; l < m.L; ++l) {
    const LayerDev& L = e->layers[l];
    QkvArgs qa{};
    qa.x = e->x;
    qa.emb = l == 0 ? e->emb : nullptr;
    qa.x_out = e->x;
    qa.st = e->st;
    qa.nw = L.rms_att; qa.eps = e->eps;
    qa.D = m.D; qa.Dq = m.Dq; qa.Dkv = m.Dkv; qa.g = e->l_qkv.g;
    qa.wq = L.wq; qa.wk = L.wk; qa.wv = L.wv; qa.bq = L.bq; qa.bk = L.bk; qa.bv = L.bv;
    qa.q_out = e->q;
    qa.kcache = e->kcache + l * kv_layer;
    qa.vcache = e->vcache + l * kv_layer;
    mark(s, mk, kKQkv);
    KL_GEMV_LAUNCH(k_qkv, Q8, e->l_qkv, s, qa);

    AttnArgs aa{};
    aa.q = e->q;
    aa.kcache = e->kcache + l * kv_layer;
    aa.vcache = e->vcache + l * kv_layer;
    aa.out = e->att;
    aa.part = e->attn_part;
    aa.counters = e->attn_counters;
    aa.pos_ptr = &e->st->pos;
    aa.kv_dim = m.Dkv;
    aa.kv_mul = m.H / m.KVH;
    aa.G = e->attn.G;
    aa.cpw = 1;
    aa.transform = e->transform;
    aa.rope_style = e->rope_style;
    aa.sin_t = e->sin_t;
    aa.cos_t = e->cos_t;
    aa.qn = L.qn;
    aa.kn = L.kn;
    aa.qk_eps = 1e-6f;  // kernels/cuda/rmsnorm_kernel.cu:148
    aa.scale = 1.f / std::sqrt(static_cast<float>(m.hd));
    const dim3 ag(m.KVH * e->attn.G);
    mark(s, mk, kKAttn);
    switch (m.hd) {
      case 32: hipLaunchKernelGGL(k_attn_decode<32>, ag, dim3(256), e->attn.lds_bytes, s, aa); break;
      case 64: hipLaunchKernelGGL(k_attn_decode<64>, ag, dim3(256), e->attn.lds_bytes, s, aa); break;
      case 128: hipLaunchKernelGGL(k_attn_decode<128>, ag, dim3(256), e->attn.lds_bytes, s, aa); break;
      default: hipLaunchKernelGGL(k_attn_decode<256>, ag, dim3(256), e->attn.lds_bytes, s, aa); break;
    }

    ResArgs ra{};
    ra.in = e->att; ra.rows = m.D; ra.g = e->l_wo.g; ra.w = L.wo; ra.x = e->x;
    mark(s, mk, kKWo);
    KL_GEMV_LAUNCH(k_gemv_residual, Q8, e->l_wo, s, ra);

    W13Args wa{};
    wa.x = e->x; wa.nw = L.rms_ffn; wa.eps = e->eps;
    wa.D = m.D; wa.F = m.F; wa.g = e->l_w13.g;
    wa.w1 = L.w1; wa.w3 = L.w3; wa.h = e->h;
    mark(s, mk, kKW13);
    KL_GEMV_LAUNCH(k_w13_swiglu, Q8, e->l_w13, s, wa);

    ResArgs rb{};
    rb.in = e->h; rb.rows = m.D; rb.g = e->l_w2.g; rb.w = L.w2; rb.x = e->x;
    mark(s, mk, kKW2);
    KL_GEMV_LAUNCH(k_gemv_residual, Q8, e->l_w2, s, rb);
  }
  ClsArgs ca{};
  ca.x = e->x; ca.nw = e->rms_final; ca.eps = e->eps;
  ca.D = m.D; ca.V = m.V; ca.g = e->l_cls.g;
  ca.w = e->wcls; ca.logits = e->logits;
  ca.pv = e->am_pv; ca.pi = e->am_pi; ca.counter = e->am_counter;
  ca.st = e->st; ca.prompt = e->prompt; ca.out_tokens = e->out_tokens;
  mark(s, mk, kKCls);
  KL_GEMV_LAUNCH(k_cls_argmax, Q8, e->l_cls, s, ca);
  mark(s, mk, kKEnd);
  return rc(hipGetLastError());
}

int launch_step(kl_engine* e, Marks* mk = nullptr) {
  return e->quant ? launch_step_t<true>(e, mk) : launch_step_t<false>(e, mk);
}

// One persistent launch = one token.
// Uploads the device step state (the next launch's position and token).
hipError_t set_state(kl_engine* e, const StepState& st) {
  *e->st_host = st;
  e->host_pos = st.pos;
  return hipMemcpyAsync(e->st, e->st_host, sizeof(StepState), hipMemcpyHostToDevice, e->stream);
}

int launch_persistent(kl_engine* e, Marks* mk = nullptr) {
  void* params[] = {&e->pargs};
  const size_t lds = e->pargs.trace ? e->p_lds_traced : e->p_lds;
  // Every launch advances the device position by one; the host follows it to
  // pick the attention variant (a mismatch is reported by the kernel).
  const void* k = e->host_pos + 1 <= e->pargs.attn_short_max ? e->p_kernel_short : e->p_kernel;
  ++e->host_pos;
  mark(e->stream, mk, kKStep);
  const hipError_t err =
      e->plain_launch
          ? hipLaunchKernel(k, dim3(e->nwg), dim3(kPThreads), params, lds, e->stream)
          : hipLaunchCooperativeKernel(k, dim3(e->nwg), dim3(kPThreads), params, lds, e->stream);
  mark(e->stream, mk, kKEnd);
  return rc(err);
}

int run_step(kl_engine* e) {
  if (e->mode == KL_MODE_PERSISTENT) return launch_persistent(e);
  if (!e->use_graph) return launch_step(e);
  if (!e->graph_exec) {
    hipError_t err = hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal);
    if (err != hipSuccess) return rc(err);
    const int lrc = launch_step(e);
    hipGraph_t g = nullptr;
    err = hipStreamEndCapture(e->stream, &g);
    if (lrc != KL_OK) {
      if (g) (void)hipGraphDestroy(g);
      return lrc;
    }
    if (err != hipSuccess) return rc(err);
    err = hipGraphInstantiate(&e->graph_exec, g, nullptr, nullptr, 0);
    if (err != hipSuccess) {
      (void)hipGraphDestroy(g);
      e->graph_exec = nullptr;
      return rc(err);
    }
    e->graph = g;
  }
  return rc(hipGraphLaunch(e->graph_exec, e->stream));
}

// Reads the device error word after the stream has been synchronised; on an
// error, resets the barrier state so the engine can be used again.
int check_device_error(kl_engine* e) {
  if (e->mode != KL_MODE_PERSISTENT) return KL_OK;
  hipError_t err = hipMemcpy(e->derr_host, e->derr, sizeof(int), hipMemcpyDeviceToHost);
  if (err != hipSuccess) return rc(err);
  if (*e->derr_host == 0) return KL_OK;
  fprintf(stderr, "kuiper_hip: persistent step reported device error %d\n", *e->derr_host);
  err = hipMemset(e->derr, 0, sizeof(int));
  if (err == hipSuccess) err = hipMemset(e->am_counter, 0, sizeof(unsigned int));
  if (err == hipSuccess) err = hipMemset(e->cls_next, 0, sizeof(unsigned int));
  if (err == hipSuccess) err = hipMemset(e->attn_counters, 0, e->lay.KVH * sizeof(unsigned int));
  if (err == hipSuccess) err = hipDeviceSynchronize();
  return err == hipSuccess ? KL_EDEVICE : rc(err);
}

// ---------------------------------------------------------------------------
// Persistent-step planning.
// ---------------------------------------------------------------------------
// Fills the geometry of one GEMV phase for segments of nb chunks: rows split
// into balanced contiguous ranges, one per workgroup, then (ks, rw) chosen to
// minimise the largest per-wave work, counting a row reduction as half a
// chunk.  Returns the LDS floats the phase's row partials need.
// The split-K factor is chosen for the balanced share, so a row's summation
// order (and so every result bit) does not depend on the measured split;
// `max_share` (the largest weighted share, or 0) only sizes the LDS slots.
size_t plan_phase(PGemv& p, int nwg, bool q8, int gs, int nb, int max_share) {
  const int total = (p.paired ? p.rows[0] : p.rows[0] + p.rows[1] + p.rows[2]) - p.dyn;
  const int rpw = (total + nwg - 1) / nwg;  // balanced per-workgroup share
  p.cn16 = q8 ? p.cols / 16 : p.cols / 4;
  p.cn = (p.cn16 + kWave - 1) / kWave;
  p.nseg = (p.cn + nb - 1) / nb;
  p.gshift = 0;
  if (q8)
    while ((1 << p.gshift) < gs) ++p.gshift;
  const int nloc = p.paired ? rpw * p.nsub : rpw;
  double best = 1e30;
  int ks_lo = 1, ks_hi = kPWaves;
  if (const char* env = std::getenv("KL_PKS")) {  // tuning: force the split-K factor
    const int v = std::atoi(env);
    if (v == 1 || v == 2 || v == 4 || v == 8) ks_lo = ks_hi = v;
  }
  for (int ks = ks_lo; ks <= ks_hi; ks *= 2) {
    const int rw = kPWaves / ks;
    const int nsegw = (p.nseg + ks - 1) / ks;
    double cost = static_cast<double>((nloc + rw - 1) / rw) * (nsegw * nb + 0.5);
    if (!q8 && nsegw == 1) cost *= 0.9;  // the input slice stays in registers
    if (cost < best - 1e-9) {
      best = cost;
      p.ks = ks;
      p.rw = rw;
      p.nsegw = nsegw;
    }
  }
  const int rmax = std::max(std::max(rpw, max_share), p.dyn > 0 ? p.blk : 0);
  return static_cast<size_t>(p.paired ? rmax * p.nsub : rmax) * p.ks;
}

template <bool Q8, int NB, bool SHORT>
const void* persistent_kernel(int hd) {
  switch (hd) {
    case 32: return reinterpret_cast<const void*>(&k_decode_persistent<Q8, NB, 32, SHORT>);
    case 64: return reinterpret_cast<const void*>(&k_decode_persistent<Q8, NB, 64, SHORT>);
    case 128: return reinterpret_cast<const void*>(&k_decode_persistent<Q8, NB, 128, SHORT>);
    default: return reinterpret_cast<const void*>(&k_decode_persistent<Q8, NB, 256, SHORT>);
  }
}

// Row offsets [nwg + 1] for `total` rows with shares proportional to w (every
// workgroup keeps at least one row: the tagged hand-off relies on it).
std::vector<int> weighted_split(int total, const std::vector<double>& w) {
  const int n = static_cast<int>(w.size());
  std::vector<int> off(n + 1, 0);
  double sum = 0.0;
  for (double x : w) sum += x;
  double acc = 0.0;
  for (int b = 0; b < n; ++b) {
    acc += w[b];
    int e = static_cast<int>(std::llround(acc / sum * total));
    e = std::max(e, off[b] + 1);              // at least one row
    e = std::min(e, total - (n - 1 - b));      // leave one for each later workgroup
    off[b + 1] = e;
  }
  off[n] = total;
  return off;
}

int max_share(const std::vector<int>& off) {
  int m = 0;
  for (size_t b = 0; b + 1 < off.size(); ++b) m = std::max(m, off[b + 1] - off[b]);
  return m;
}

// Builds the phase descriptors and launch shape; leaves persistent_ok false
// (and the multi-kernel mode selected) where the device cannot hold the grid.
int setup_persistent(kl_engine* e) {
  const ImageLayout& m = e->lay;
  const bool q8 = e->quant != 0;
  // Hand-off tags are epoch * kTagLayers + layer + 1 for layers -1 .. L-1:
  // with L >= kTagLayers one launch's last layer would carry the next
  // launch's first tag, so such models run the multi-kernel step.
  if (m.L >= kTagLayers) return KL_OK;
  int nb = 4;
  if (const char* env = std::getenv("KL_PNB")) nb = std::atoi(env);
  if (q8) {
    e->p_kernel = nb == 4 ? persistent_kernel<true, 4, false>(m.hd) : persistent_kernel<true, 8, false>(m.hd);
    e->p_kernel_short = nb == 4 ? persistent_kernel<true, 4, true>(m.hd) : persistent_kernel<true, 8, true>(m.hd);
  } else {
    e->p_kernel = nb == 4 ? persistent_kernel<false, 4, false>(m.hd) : persistent_kernel<false, 8, false>(m.hd);
    e->p_kernel_short = nb == 4 ? persistent_kernel<false, 4, true>(m.hd) : persistent_kernel<false, 8, true>(m.hd);
  }
  if (nb != 4 && nb != 8) nb = 8;
  int per_cu = 1;
  if (const char* env = std::getenv("KL_PWG_PER_CU"))
    per_cu = std::min(kMaxPwgPerCu, std::max(1, std::atoi(env)));
  // Every workgroup must own at least one row of every GEMV phase (the
  // dataflow hand-off relies on it), so the grid is capped at the smallest
  // phase's row count.
  const int min_rows = std::min(std::min(m.D, m.F), std::min(m.Dq + 2 * m.Dkv, m.V));
  e->nwg = std::min(e->cus * per_cu, min_rows);
  std::vector<PGemv> ph(4 * m.L + 1);
  std::vector<PAttn> at(m.L);
  size_t red_floats = 0;
  int max_cols = 0;
  for (int l = 0; l < m.L; ++l) {
    const LayerDev& L = e->layers[l];
    const size_t kv_layer = static_cast<size_t>(m.S) * m.Dkv;
    PGemv& qkv = ph[4 * l + 0];
    qkv = PGemv{};
    qkv.w[0] = L.wq.w; qkv.w[1] = L.wk.w; qkv.w[2] = L.wv.w;
    qkv.sc[0] = L.wq.s; qkv.sc[1] = L.wk.s; qkv.sc[2] = L.wv.s;
    qkv.rows[0] = m.Dq; qkv.rows[1] = m.Dkv; qkv.rows[2] = m.Dkv;
    qkv.nsub = 3; qkv.paired = 0; qkv.cols = m.D; qkv.epi = kEpiQkv;
    qkv.layer = l; qkv.in_layer = l - 1;
    qkv.in = l == 0 ? nullptr : e->t_x;
    qkv.norm = L.rms_att;
    qkv.out[0] = e->t_q; qkv.out[1] = e->t_k; qkv.out[2] = e->t_v;
    qkv.vcache = e->vcache + l * kv_layer;
    qkv.bias[0] = L.bq; qkv.bias[1] = L.bk; qkv.bias[2] = L.bv;
    PGemv& wo = ph[4 * l + 1];
    wo = PGemv{};
    wo.w[0] = L.wo.w; wo.sc[0] = L.wo.s; wo.rows[0] = m.D;
    wo.nsub = 1; wo.cols = m.Dq; wo.epi = kEpiResid;
    wo.layer = l; wo.in_layer = l;
    wo.in = e->t_att; wo.norm = nullptr; wo.out[0] = e->t_xb;
    PGemv& w13 = ph[4 * l + 2];
    w13 = PGemv{};
    w13.w[0] = L.w1.w; w13.w[1] = L.w3.w; w13.sc[0] = L.w1.s; w13.sc[1] = L.w3.s;
    w13.rows[0] = m.F; w13.rows[1] = m.F;
    w13.nsub = 2; w13.paired = 1; w13.cols = m.D; w13.epi = kEpiSwiglu;
    w13.layer = l; w13.in_layer = l;
    w13.in = e->t_xb; w13.norm = L.rms_ffn; w13.out[0] = e->t_h;
    PGemv& w2 = ph[4 * l + 3];
    w2 = PGemv{};
    w2.w[0] = L.w2.w; w2.sc[0] = L.w2.s; w2.rows[0] = m.D;
    w2.nsub = 1; w2.cols = m.F; w2.epi = kEpiResid;
    w2.layer = l; w2.in_layer = l;
    w2.in = e->t_h; w2.norm = nullptr; w2.out[0] = e->t_x;
    at[l] = PAttn{e->kcache + l * kv_layer, e->vcache + l * kv_layer, L.qn, L.kn};
  }
  // The classifier's last rows are handed out at run time in blocks, so that
  // workgroups that finish their static share early take more: the slowest
  // workgroup otherwise ends the step ~10 us after the median one.  Measured:
  // 20 % in blocks of 16 rows +0.7% on Llama-3.2-1B (4 MB of classifier per
  // workgroup; 10 %: +-0, 40 %: -0.2%), +-0 on Qwen2.5-1.5B and Qwen3-4B,
  // -1% on Llama2-110M (0.4 MB per workgroup, whose tail is short anyway), so
  // it is on from 2 MB of classifier weights per workgroup.
  // KL_CLS_DYN: percent of the rows (0: off); KL_CLS_BLOCK: rows per block.
  const double cls_bytes_wg = static_cast<double>(m.V) * m.D * (q8 ? 1.0 + 4.0 / m.gs : 4.0) / e->nwg;
  int cls_blk = 16, cls_pct = cls_bytes_wg >= 2.0 * (1 << 20) ? 20 : 0;
  if (const char* env = std::getenv("KL_CLS_BLOCK")) cls_blk = std::max(1, std::atoi(env));
  if (const char* env = std::getenv("KL_CLS_DYN")) cls_pct = std::min(90, std::max(0, std::atoi(env)));
  int cls_dyn = static_cast<int>(static_cast<long long>(m.V) * cls_pct / 100);
  if (m.V - cls_dyn < e->nwg) cls_dyn = 0;  // every workgroup keeps a static row
  // Weighted splits (after calibration) for the four split dimensions.
  const bool weighted = static_cast<int>(e->wg_weight.size()) == e->nwg;
  int share_qkv = 0, share_d = 0, share_f = 0, share_v = 0;
  if (weighted) {
    const std::vector<int> sq = weighted_split(m.Dq + 2 * m.Dkv, e->wg_weight);
    const std::vector<int> sd = weighted_split(m.D, e->wg_weight);
    const std::vector<int> sf = weighted_split(m.F, e->wg_weight);
    const std::vector<int> sv = weighted_split(m.V - cls_dyn, e->wg_weight);
    share_qkv = max_share(sq);
    share_d = max_share(sd);
    share_f = max_share(sf);
    share_v = max_share(sv);
    const size_t per = static_cast<size_t>(e->nwg) + 1;
    if (!e->d_split) {
      hipError_t err = hipMalloc(&e->d_split, 4 * per * sizeof(int));
      if (err != hipSuccess) return rc(err);
    }
    std::vector<int> all;
    for (const auto* t : {&sq, &sd, &sf, &sv}) all.insert(all.end(), t->begin(), t->end());
    hipError_t err = hipMemcpy(e->d_split, all.data(), all.size() * sizeof(int), hipMemcpyHostToDevice);
    if (err != hipSuccess) return rc(err);
    for (int l = 0; l < m.L; ++l) {
      ph[4 * l + 0].split = e->d_split;
      ph[4 * l + 1].split = e->d_split + per;
      ph[4 * l + 2].split = e->d_split + 2 * per;
      ph[4 * l + 3].split = e->d_split + per;
    }
  }
  PGemv& cls = ph[4 * m.L];
  cls = PGemv{};
  cls.w[0] = e->wcls.w; cls.sc[0] = e->wcls.s; cls.rows[0] = m.V;
  cls.nsub = 1; cls.cols = m.D; cls.epi = kEpiCls;
  cls.dyn = cls_dyn; cls.blk = cls_blk;
  cls.layer = m.L - 1; cls.in_layer = m.L - 1;
  cls.in = e->t_x; cls.norm = e->rms_final; cls.logits = e->logits;
  if (weighted) cls.split = e->d_split + 3 * (static_cast<size_t>(e->nwg) + 1);
  for (size_t i = 0; i < ph.size(); ++i) {
    PGemv& p = ph[i];
    int share = 0;
    if (weighted) {
      if (i + 1 == ph.size()) share = share_v;         // classifier
      else if (i % 4 == 0) share = share_qkv;          // QKV
      else if (i % 4 == 2) share = share_f;            // W1/W3
      else share = share_d;                            // WO, W2
    }
    red_floats = std::max(red_floats, plan_phase(p, e->nwg, q8, m.gs, nb, share));
    max_cols = std::max(max_cols, p.cols);
  }
  const int red_off = ((q8 ? xpad(max_cols) : max_cols) + 3) & ~3;  // int8: padded input layout
  const int xres_off = red_off + static_cast<int>((red_floats + 3) & ~size_t(3));
  const int xres_floats = weighted ? share_d : (m.D + e->nwg - 1) / e->nwg;
  const size_t gemv_lds = (static_cast<size_t>(xres_off) + xres_floats) * sizeof(float);
  const size_t attn_lds = std::max(attn_p_lds_floats(m.hd, m.H / m.KVH),
                                   attn_short_lds_floats(m.hd)) * sizeof(float);
  // The residual rows must survive the attention phase, which uses LDS from 0.
  const size_t xres_at = std::max(static_cast<size_t>(xres_off) * sizeof(float),
                                  (attn_lds + 15) & ~size_t(15));
  e->p_lds = xres_at + xres_floats * sizeof(float);
  (void)gemv_lds;
  const int trace_slots = 2 * 5 * m.L + 3;
  const size_t trace_at = (e->p_lds + 15) & ~size_t(15);
  e->p_lds_traced = trace_at + trace_slots * sizeof(unsigned long long);
  hipError_t err = hipMemcpy(e->d_ph, ph.data(), ph.size() * sizeof(PGemv), hipMemcpyHostToDevice);
  if (err == hipSuccess)
    err = hipMemcpy(e->d_at, at.data(), at.size() * sizeof(PAttn), hipMemcpyHostToDevice);
  if (err != hipSuccess) return rc(err);

  PArgs& a = e->pargs;
  a = PArgs{};
  a.ph = e->d_ph; a.at = e->d_at;
  a.L = m.L; a.D = m.D; a.Dq = m.Dq; a.Dkv = m.Dkv; a.V = m.V; a.S = m.S;
  a.kv_mul = m.H / m.KVH; a.KVH = m.KVH;
  a.eps = e->eps; a.qk_eps = 1e-6f;  // kernels/cuda/rmsnorm_kernel.cu:148
  a.scale = 1.f / std::sqrt(static_cast<float>(m.hd));
  a.rope_style = e->rope_style; a.transform = e->transform;
  a.sin_t = e->sin_t; a.cos_t = e->cos_t; a.emb = e->emb;
  a.q = e->t_q; a.knew = e->t_k; a.vnew = e->t_v; a.att = e->t_att;
  a.attn_part = e->t_part;
  a.attn_part_n = static_cast<long long>(e->attn.part_floats);
  a.attn_G = e->attn.G;
  // Attention merge beyond kAttnMergeChunks chunks per kv head: one merging
  // workgroup per 2 chunks (measured best of 1, 2, 4, 8 on Qwen2.5-1.5B at
  // 4000 positions; KL_ATTN_MERGE_CHUNKS overrides).
  a.merge_chunks = 2;
  if (const char* env = std::getenv("KL_ATTN_MERGE_CHUNKS")) a.merge_chunks = std::max(1, std::atoi(env));
  // 9-16 chunks: a merger per 4 chunks (3-4 per kv head) measured +1.4%
  // on Qwen3-4B at 520-640 positions and +0.6% on Llama-3.2-1B at 600-700
  // against one per 2; beyond 16 chunks one per 2 stays best (Qwen2.5-1.5B
  // at 4000 positions: one per 4 -1.1%).
  a.merge_chunks_mid = 4;
  if (const char* env = std::getenv("KL_ATTN_MERGE_CHUNKS_MID"))
    a.merge_chunks_mid = std::max(1, std::atoi(env));
  // While the attention runs, workgroups without an attention item pull the
  // first 96 KB (up to 1.5x with many attention items) of their W1/W3 rows into L2 (those of the XCD's attention
  // workgroups are shared out among them), 0.5 us after the attention starts,
  // so that the W1/W3 stream starts from L2 instead of waiting out the HBM
  // latency.  Measured on Llama-3.2-1B at position 200 (tok/s against no
  // touch): 64 KB +2.0%, 80 KB +2.4%, 96 KB +2.5-2.8%, 112 KB +2.3%, 128 KB
  // +2.6%; delays 0 / 0.25 / 0.5 / 1 us within 0.5% of each other.  Pulling
  // the whole WO share instead gained 0.8%, and less together with W1/W3.
  // Off when a workgroup's W1/W3 share is under 128 KB (Llama2-110M: 48 KB,
  // -1%): its stream is too short for the start to matter.
  const int w13_cols_bytes = m.D * (e->quant ? 1 : 4);
  const double w13_share = 2.0 * m.F * w13_cols_bytes / e->nwg;
  a.w13_touch_rows = w13_share >= 131072.0 ? std::max(1, 98304 / w13_cols_bytes) : 0;
  a.touch_delay = 50;
  if (const char* env = std::getenv("KL_W13_TOUCH_ROWS")) a.w13_touch_rows = std::max(0, std::atoi(env));
  if (const char* env = std::getenv("KL_TOUCH_DELAY")) a.touch_delay = std::max(0, std::atoi(env));
  // Short-context attention (one item per query head, no merge) up to the
  // positions its registers hold; KL_ATTN_SHORT_MAX lowers the limit (0: off).
  a.attn_short_max = attn_short_rows(m.hd);
  if (const char* env = std::getenv("KL_ATTN_SHORT_MAX"))
    a.attn_short_max = std::min(a.attn_short_max, std::max(0, std::atoi(env)));
  a.short_touch_rows = a.w13_touch_rows;
  // Inputs at least this wide are staged two elements per load (measured:
  // +1.1-1.3% on Llama-3.2-1B, Llama2-7B int8 and Qwen2.5-1.5B from the
  // 8192- to 11008-wide W2 inputs; narrower inputs measured slower paired).
  a.stage_pair_min = 4096;
  if (const char* env = std::getenv("KL_STAGE_PAIR_MIN")) a.stage_pair_min = std::max(2, std::atoi(env));
  a.kc0 = e->kcache;
  a.vc0 = e->vcache;
  a.kv_layer = static_cast<long long>(m.S) * m.Dkv;
  a.qkn = e->qkn;
  if (const char* env = std::getenv("KL_W13_TOUCH_ROWS_SHORT"))
    a.short_touch_rows = std::max(0, std::atoi(env));
  a.am_pv = e->am_pv; a.am_pi = e->am_pi; a.am_cnt = e->am_counter;
  a.cls_next = e->cls_next;
  a.epoch = e->epoch; a.err = e->derr;
  a.red_off = red_off;
  a.xres_off = static_cast<int>(xres_at / sizeof(float));
  a.st = e->st; a.prompt = e->prompt; a.out_tokens = e->out_tokens;
  a.trace_off = static_cast<int>(trace_at / sizeof(unsigned long long));
  a.trace_slots = trace_slots;

  // The grid must be co-resident: one workgroup of 512 threads per CU (or
  // KL_PWG_PER_CU) with this LDS.
  int blocks = kMaxPwgPerCu;
  e->trace_ok = true;
  for (const void* kern : {e->p_kernel, e->p_kernel_short}) {
    if (e->p_lds_traced > 64 * 1024) {
      err = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(e->p_lds_traced));
      if (err != hipSuccess) {
        (void)hipGetLastError();
        return KL_OK;
      }
    }
    int b = 0;
    err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, kern, kPThreads, e->p_lds);
    if (err != hipSuccess) {
      (void)hipGetLastError();
      return KL_OK;
    }
    blocks = std::min(blocks, b);
    int bt = 0;
    e->trace_ok = e->trace_ok &&
                  hipOccupancyMaxActiveBlocksPerMultiprocessor(&bt, kern, kPThreads, e->p_lds_traced) ==
                      hipSuccess &&
                  bt >= per_cu;
  }
  e->persistent_ok = blocks >= per_cu;
  (void)hipGetLastError();
  e->mode = e->persistent_ok ? KL_MODE_PERSISTENT : KL_MODE_MULTI;
  e->plain_launch = e->persistent_ok && blocks * e->cus >= e->nwg;
  if (const char* env = std::getenv("KL_PERSISTENT_LAUNCH"))
    if (std::strcmp(env, "cooperative") == 0) e->plain_launch = false;
  if (const char* env = std::getenv("KL_ENGINE_MODE")) {
    if (std::atoi(env) == KL_MODE_MULTI) e->mode = KL_MODE_MULTI;
  }
  return KL_OK;
}

void release(kl_engine* e) {
  if (!e) return;
  if (e->graph_exec) (void)hipGraphExecDestroy(e->graph_exec);
  if (e->graph) (void)hipGraphDestroy(e->graph);
  if (e->ev0) (void)hipEventDestroy(e->ev0);
  if (e->ev1) (void)hipEventDestroy(e->ev1);
  if (e->arena) (void)hipFree(e->arena);
  if (e->pf_buf) (void)hipFree(e->pf_buf);
  if (e->xw_buf) (void)hipFree(e->xw_buf);
  if (e->d_split) (void)hipFree(e->d_split);
  if (e->st_host) (void)hipHostFree(e->st_host);
  if (e->derr_host) (void)hipHostFree(e->derr_host);
  if (e->stream) (void)hipStreamDestroy(e->stream);
  delete e;
}

}  // namespace

namespace {

// One traced persistent step (token, pos): ticks [2 * 5 * L + 3][nwg].
int trace_once(kl_engine* e, int32_t token, int32_t pos, unsigned long long* ticks) {
  if (!e->trace_ok) return KL_EUNSUPP;
  const size_t n = static_cast<size_t>(2 * 5 * e->lay.L + 3) * e->nwg;
  unsigned long long* d = nullptr;
  hipError_t err = hipMalloc(&d, n * sizeof(unsigned long long));
  if (err != hipSuccess) return rc(err);
  err = hipMemset(d, 0, n * sizeof(unsigned long long));
  if (err == hipSuccess) err = set_state(e, StepState{pos, token, 0, 0});
  int r = rc(err);
  if (r == KL_OK) {
    e->pargs.trace = d;
    r = launch_persistent(e);
    e->pargs.trace = nullptr;
  }
  if (r == KL_OK) r = rc(hipStreamSynchronize(e->stream));
  if (r == KL_OK) r = check_device_error(e);
  if (r == KL_OK) r = rc(hipMemcpy(ticks, d, n * sizeof(unsigned long long), hipMemcpyDeviceToHost));
  (void)hipFree(d);
  return r;
}

// Measures each workgroup's time on the W1/W3 and W2 phases (the bulk of the
// streaming) over a few traced steps and re-splits every phase's rows in
// proportion to the workgroups' speed.  On MI355X some XCDs stream a few
// percent slower than others, and which ones differs between parts, so the
// split is measured rather than fixed.  Results do not change (the split-K
// plan stays the balanced one).  KL_PCALIBRATE=0 keeps the balanced split.
int calibrate_persistent(kl_engine* e) {
  if (!e->persistent_ok || !e->trace_ok || e->mode != KL_MODE_PERSISTENT) return KL_OK;
  // Passes of the fixed-point iteration (KL_PCALIBRATE; 0 disables): each
  // re-measures the FFN phases with the current split and scales every
  // workgroup's weight by mean work / its work.  One pass: a second evens out
  // the per-XCD means further but does not lower the slowest workgroup, whose
  // identity varies from step to step (measured).
  int passes = 1;
  if (const char* env = std::getenv("KL_PCALIBRATE")) passes = std::max(0, std::atoi(env));
  const int L = e->lay.L, W = e->nwg;
  if (e->lay.S < 4 || passes == 0) return KL_OK;
  std::vector<unsigned long long> t(static_cast<size_t>(2 * 5 * L + 3) * W);
  std::vector<double> wt(W, 1.0);
  for (int pass = 0; pass < passes; ++pass) {
    std::vector<double> work(W, 0.0);
    for (int rep = 0; rep < 4; ++rep) {
      const int r = trace_once(e, 0, rep, t.data());
      if (r != KL_OK) return r;
      if (rep == 0) continue;  // warm-up
      for (int l = 0; l < L; ++l)
        for (int p : {5 * l + 3, 5 * l + 4}) {  // W1/W3, W2
          const unsigned long long* ready = t.data() + static_cast<size_t>(2 * p + 1) * W;
          const unsigned long long* done = t.data() + static_cast<size_t>(2 * p + 2) * W;
          for (int b = 0; b < W; ++b)
            work[b] += done[b] > ready[b] ? static_cast<double>(done[b] - ready[b]) : 0.0;
        }
    }
    double mean = 0.0;
    for (double w : work) mean += w;
    mean /= W;
    if (!(mean > 0.0)) return KL_OK;
    for (int b = 0; b < W; ++b) {
      const double sp = work[b] > 0.0 ? mean / work[b] : 1.0;  // relative speed
      wt[b] = std::min(1.25, std::max(0.8, wt[b] * sp));
    }
    e->wg_weight = wt;
    const int r = setup_persistent(e);
    if (r != KL_OK) return r;
  }
  return KL_OK;
}

}  // namespace

extern "C" {

int kl_engine_create(const void* image, size_t bytes, int family, int quant, kl_engine** out) {
  if (!out) return KL_EINVAL;
  *out = nullptr;
  ImageLayout lay;
  int prc = parse_image(image, bytes, family, quant, &lay);
  if (prc != KL_OK) return prc;
  const int kv_mul = lay.H / lay.KVH;
  if (!mha_shape_ok(lay.H, kv_mul, lay.hd)) return KL_EUNSUPP;
  if (lay.D % 4 != 0 || lay.Dq % 4 != 0 || lay.F % 4 != 0) return KL_EUNSUPP;
  int chunk_shift = 0;
  if (quant) {
    const int cpg = lay.gs / 16;
    if (lay.gs % 16 != 0 || (cpg & (cpg - 1)) != 0 || lay.D % lay.gs != 0 ||
        lay.Dq % lay.gs != 0 || lay.F % lay.gs != 0)
      return KL_EUNSUPP;
    while ((1 << chunk_shift) < cpg) ++chunk_shift;
  }

  kl_engine* e = new kl_engine();
  e->lay = lay;
  e->family = family;
  e->quant = quant;
  e->chunk_shift = chunk_shift;
  switch (family) {
    case KL_FAMILY_LLAMA2: e->eps = 1e-5f; e->theta = 10000.f; e->rope_style = KL_ROPE_INTERLEAVED; break;
    case KL_FAMILY_LLAMA3: e->eps = 1e-5f; e->theta = 500000.f; e->rope_style = KL_ROPE_HALF; break;
    case KL_FAMILY_QWEN2: e->eps = 1e-6f; e->theta = 1000000.f; e->rope_style = KL_ROPE_HALF; break;
    default: e->eps = 1e-6f; e->theta = 1000000.f; e->rope_style = KL_ROPE_HALF; break;
  }
  e->transform = family == KL_FAMILY_QWEN3 ? 2 : 1;
  {
    // Batched prefill of fp32 images with every GEMM depth a multiple of 32:
    // split-product GEMMs; KL_PREFILL_GEMM=f32 keeps the fp32 matrix-core kernels.
    const char* env = std::getenv("KL_PREFILL_GEMM");
    e->pf_x6 = !quant && lay.D % 32 == 0 && lay.Dq % 32 == 0 && lay.F % 32 == 0 &&
               !(env && std::strcmp(env, "f32") == 0);
    const int gs = lay.gs;
    e->pf_q8s = quant && (gs == 32 || gs == 64) && lay.D % gs == 0 && lay.Dq % gs == 0 &&
                lay.F % gs == 0 && !(env && std::strcmp(env, "f32") == 0);
  }
  int dev = 0;
  hipDeviceProp_t prop;
  if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
    e->cus = prop.multiProcessorCount;
  e->grid_cap = e->cus * 2;
  if (const char* env = std::getenv("KL_GRID_PER_CU")) {
    const int v = std::atoi(env);
    if (v > 0) e->grid_cap = e->cus * v;
  }
  e->attn = mha_plan(lay.KVH, kv_mul, lay.S, lay.hd);
  if (e->attn.G > 512) {
    delete e;
    return KL_EUNSUPP;  // the chunk merge keeps (m, l) of at most 512 chunks in LDS
  }
  e->l_qkv = plan_gemv(e, lay.Dq + 2 * lay.Dkv, lay.D);
  e->l_wo = plan_gemv(e, lay.D, lay.Dq);
  e->l_w13 = plan_gemv(e, lay.F, lay.D);
  e->l_w2 = plan_gemv(e, lay.D, lay.F);
  e->l_cls = plan_gemv(e, lay.V, lay.D);
  for (const auto* L : {&e->l_qkv, &e->l_wo, &e->l_w13, &e->l_w2, &e->l_cls}) {
    if (L->g.ks > kMaxKs) {
      delete e;
      return KL_EUNSUPP;
    }
  }

  // Arena plan: every tensor 256-byte aligned.
  size_t cursor = 0;
  auto plan = [&](size_t bytes) {
    const size_t at = cursor;
    cursor += (bytes + 255) & ~size_t(255);
    return at;
  };
  struct Slot {
    const HostTensor* src;
    size_t at;
  };
  std::vector<Slot> slots;
  auto place = [&](const HostTensor& t) -> size_t {
    if (!t.ptr) return SIZE_MAX;
    const size_t at = plan(t.bytes);
    slots.push_back({&t, at});
    return at;
  };
  struct LayerOff {
    size_t rms_att, rms_ffn, bq, bk, bv, qn, kn, wq, wk, wv, wo, w1, w2, w3, sq, sk, sv, so, s1, s2,
        s3;
  };
  const size_t emb_at = place(e->lay.emb);
  const size_t fin_at = place(e->lay.rms_final);
  const size_t cls_at = e->lay.wcls.ptr ? place(e->lay.wcls) : SIZE_MAX;
  const size_t scls_at = e->lay.scls.ptr ? place(e->lay.scls) : SIZE_MAX;
  std::vector<LayerOff> lo(lay.L);
  for (int l = 0; l < lay.L; ++l) {
    const LayerHost& H = e->lay.layers[l];
    LayerOff& o = lo[l];
    o.rms_att = place(H.rms_att); o.rms_ffn = place(H.rms_ffn);
    o.bq = place(H.bq); o.bk = place(H.bk); o.bv = place(H.bv);
    o.qn = place(H.qn); o.kn = place(H.kn);
    o.wq = place(H.wq); o.wk = place(H.wk); o.wv = place(H.wv); o.wo = place(H.wo);
    o.w1 = place(H.w1); o.w2 = place(H.w2); o.w3 = place(H.w3);
    o.sq = place(H.sq); o.sk = place(H.sk); o.sv = place(H.sv); o.so = place(H.so);
    o.s1 = place(H.s1); o.s2 = place(H.s2); o.s3 = place(H.s3);
  }
  size_t wbytes = 0;
  for (const Slot& sl : slots) wbytes += sl.src->bytes;
  e->weight_bytes = wbytes;
  const size_t S = lay.S, Dkv = lay.Dkv;
  const size_t sin_at = plan(S * lay.hd * 4), cos_at = plan(S * lay.hd * 4);
  const size_t kc_at = plan(static_cast<size_t>(lay.L) * S * Dkv * 4);
  const size_t vc_at = plan(static_cast<size_t>(lay.L) * S * Dkv * 4);
  const size_t x_at = plan(lay.D * 4), q_at = plan(lay.Dq * 4), att_at = plan(lay.Dq * 4);
  const size_t h_at = plan(static_cast<size_t>(lay.F) * 4), lg_at = plan(static_cast<size_t>(lay.V) * 4);
  const size_t part_at = plan(e->attn.part_floats * 4);
  // Zero-initialised region: counters and state.
  const size_t zero_begin = cursor;
  const size_t actr_at = plan(lay.KVH * sizeof(unsigned int));
  const size_t amc_at = plan(64);
  const size_t st_at = plan(sizeof(StepState));
  const size_t epoch_at = plan(sizeof(unsigned int));
  const size_t derr_at = plan(sizeof(int));
  // Tagged hand-off vectors: zeroed, so no stale element carries a live tag.
  const size_t tq_at = plan(static_cast<size_t>(lay.Dq) * 8);
  const size_t tk_at = plan(static_cast<size_t>(lay.Dkv) * 8);
  const size_t tv_at = plan(static_cast<size_t>(lay.Dkv) * 8);
  const size_t tatt_at = plan(static_cast<size_t>(lay.Dq) * 8);
  const size_t txb_at = plan(static_cast<size_t>(lay.D) * 8);
  const size_t th_at = plan(static_cast<size_t>(lay.F) * 8);
  const size_t tx_at = plan(static_cast<size_t>(lay.D) * 8);
  const size_t tpart_at = plan(e->attn.part_floats * 8);
  const size_t zero_end = cursor;
  const int gmax = std::max(e->grid_cap, e->cus * kMaxPwgPerCu);
  const size_t ph_at = plan((4 * static_cast<size_t>(lay.L) + 1) * sizeof(PGemv));
  const size_t at_at = plan(static_cast<size_t>(lay.L) * sizeof(PAttn));
  const size_t qkn_at = plan(static_cast<size_t>(lay.L) * 2 * lay.hd * 4);  // [L][q, k][hd]
  const size_t pv_at = plan(gmax * 4), pi_at = plan(gmax * 4);
  const size_t pr_at = plan(S * 4), ot_at = plan(S * 4);
  e->arena_bytes = cursor;

  hipError_t err = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking);
  if (err == hipSuccess) err = hipMalloc(&e->arena, e->arena_bytes);
  if (err != hipSuccess) {
    (void)hipGetLastError();
    release(e);
    return err == hipErrorOutOfMemory ? KL_ENOMEM : rc(err);
  }
  for (const Slot& sl : slots) {
    err = hipMemcpy(e->arena + sl.at, sl.src->ptr, sl.src->bytes, hipMemcpyHostToDevice);
    if (err != hipSuccess) {
      release(e);
      return rc(err);
    }
  }
  auto P = [&](size_t at) -> char* { return at == SIZE_MAX ? nullptr : e->arena + at; };
  auto PF = [&](size_t at) { return reinterpret_cast<float*>(P(at)); };
  e->emb = PF(emb_at);
  e->rms_final = PF(fin_at);
  if (quant) {
    e->wcls = WView{P(cls_at), PF(scls_at)};
  } else {
    e->wcls = WView{lay.tied ? static_cast<const void*>(e->emb) : P(cls_at), nullptr};
  }
  e->layers.resize(lay.L);
  for (int l = 0; l < lay.L; ++l) {
    const LayerOff& o = lo[l];
    LayerDev& d = e->layers[l];
    d.rms_att = PF(o.rms_att); d.rms_ffn = PF(o.rms_ffn);
    d.bq = PF(o.bq); d.bk = PF(o.bk); d.bv = PF(o.bv);
    d.qn = PF(o.qn); d.kn = PF(o.kn);
    d.wq = WView{P(o.wq), PF(o.sq)}; d.wk = WView{P(o.wk), PF(o.sk)};
    d.wv = WView{P(o.wv), PF(o.sv)}; d.wo = WView{P(o.wo), PF(o.so)};
    d.w1 = WView{P(o.w1), PF(o.s1)}; d.w2 = WView{P(o.w2), PF(o.s2)};
    d.w3 = WView{P(o.w3), PF(o.s3)};
  }
  e->sin_t = PF(sin_at);
  e->cos_t = PF(cos_at);
  e->kcache = PF(kc_at);
  e->vcache = PF(vc_at);
  e->x = PF(x_at);
  e->q = PF(q_at);
  e->att = PF(att_at);
  e->h = PF(h_at);
  e->logits = PF(lg_at);
  e->attn_part = PF(part_at);
  e->attn_counters = reinterpret_cast<unsigned int*>(P(actr_at));
  e->am_counter = reinterpret_cast<unsigned int*>(P(amc_at));
  e->cls_next = e->am_counter + 8;
  e->st = reinterpret_cast<StepState*>(P(st_at));
  e->am_pv = PF(pv_at);
  e->am_pi = reinterpret_cast<int*>(P(pi_at));
  e->prompt = reinterpret_cast<int32_t*>(P(pr_at));
  e->out_tokens = reinterpret_cast<int32_t*>(P(ot_at));
  e->epoch = reinterpret_cast<unsigned int*>(P(epoch_at));
  e->derr = reinterpret_cast<int*>(P(derr_at));
  auto PT = [&](size_t at) { return reinterpret_cast<tagged_t*>(P(at)); };
  e->t_q = PT(tq_at); e->t_k = PT(tk_at); e->t_v = PT(tv_at); e->t_att = PT(tatt_at);
  e->t_xb = PT(txb_at); e->t_h = PT(th_at); e->t_x = PT(tx_at);
  e->t_part = PT(tpart_at);
  e->d_ph = reinterpret_cast<PGemv*>(P(ph_at));
  e->d_at = reinterpret_cast<PAttn*>(P(at_at));
  // The Qwen3 q/k norm weights again, side by side per layer, for the decode
  // step's short-context attention (addressed by arithmetic).
  e->qkn = PF(qkn_at);
  for (int l = 0; l < lay.L && err == hipSuccess; ++l) {
    const LayerDev& d = e->layers[l];
    float* dst = e->qkn + static_cast<size_t>(l) * 2 * lay.hd;
    if (d.qn) err = hipMemcpy(dst, d.qn, lay.hd * 4, hipMemcpyDeviceToDevice);
    if (err == hipSuccess && d.kn) err = hipMemcpy(dst + lay.hd, d.kn, lay.hd * 4, hipMemcpyDeviceToDevice);
  }
  if (err != hipSuccess) {
    release(e);
    return rc(err);
  }
  e->lay.layers.clear();  // host pointers are no longer needed
  err = hipMemset(e->arena + zero_begin, 0, zero_end - zero_begin);
  if (err == hipSuccess) err = hipMemset(e->kcache, 0, 2 * static_cast<size_t>(lay.L) * S * Dkv * 4);
  if (err == hipSuccess) err = hipHostMalloc(reinterpret_cast<void**>(&e->st_host), sizeof(StepState), hipHostMallocDefault);
  if (err == hipSuccess) err = hipHostMalloc(reinterpret_cast<void**>(&e->derr_host), sizeof(int), hipHostMallocDefault);
  if (err == hipSuccess) err = hipEventCreate(&e->ev0);
  if (err == hipSuccess) err = hipEventCreate(&e->ev1);
  if (const char* env = std::getenv("KL_EPOCH_START")) {
    // Test hook: start the tag epoch just before its wrap.
    const unsigned int ep = static_cast<unsigned int>(std::strtoul(env, nullptr, 10)) % kEpochWrap;
    if (err == hipSuccess) err = hipMemcpy(e->epoch, &ep, sizeof(ep), hipMemcpyHostToDevice);
  }
  if (err != hipSuccess) {
    release(e);
    return rc(err);
  }
  int trc = kl_sincos_table(lay.hd, lay.S, e->theta, e->sin_t, e->cos_t);
  if (trc == KL_OK) trc = setup_persistent(e);
  if (trc == KL_OK) trc = calibrate_persistent(e);
  if (trc != KL_OK) {
    release(e);
    return trc;
  }
  *out = e;
  return KL_OK;
}

int kl_engine_destroy(kl_engine* e) {
  if (!e) return KL_EINVAL;
  (void)hipStreamSynchronize(e->stream);
  release(e);
  return KL_OK;
}

int kl_engine_dims(const kl_engine* e, int32_t* o) {
  if (!e || !o) return KL_EINVAL;
  const ImageLayout& m = e->lay;
  o[0] = m.D; o[1] = m.Dq; o[2] = m.Dkv; o[3] = m.F; o[4] = m.L;
  o[5] = m.H; o[6] = m.KVH; o[7] = m.V; o[8] = m.S; o[9] = m.hd;
  return KL_OK;
}

int kl_engine_weight_bytes(const kl_engine* e, int64_t* bytes) {
  if (!e || !bytes) return KL_EINVAL;
  *bytes = static_cast<int64_t>(e->weight_bytes);
  return KL_OK;
}

int kl_engine_set_mode(kl_engine* e, int mode) {
  if (!e) return KL_EINVAL;
  if (mode == KL_MODE_PERSISTENT) {
    if (!e->persistent_ok) return KL_EUNSUPP;
  } else if (mode != KL_MODE_MULTI) {
    return KL_EINVAL;
  }
  const hipError_t err = hipStreamSynchronize(e->stream);
  if (err != hipSuccess) return rc(err);
  e->mode = mode;
  return KL_OK;
}

int kl_engine_get_mode(const kl_engine* e, int* mode) {
  if (!e || !mode) return KL_EINVAL;
  *mode = e->mode;
  return KL_OK;
}

int kl_engine_launch_shape(const kl_engine* e, int32_t* workgroups, int32_t* threads,
                           int64_t* lds_bytes) {
  if (!e) return KL_EINVAL;
  if (workgroups) *workgroups = e->nwg;
  if (threads) *threads = kPThreads;
  if (lds_bytes) *lds_bytes = static_cast<int64_t>(e->p_lds);
  return KL_OK;
}

int kl_engine_set_graph(kl_engine* e, int enable) {
  if (!e) return KL_EINVAL;
  e->use_graph = enable != 0;
  return KL_OK;
}

int kl_engine_step(kl_engine* e, int32_t token, int32_t pos, int32_t* next, float* logits) {
  if (!e) return KL_EINVAL;
  if (pos < 0 || pos >= e->lay.S) return KL_EINVAL;
  if (token < 0 || token >= e->lay.V) return KL_ETOKEN;
  hipError_t err = set_state(e, StepState{pos, token, 0, 0});
  if (err != hipSuccess) return rc(err);
  const int r = run_step(e);
  if (r != KL_OK) return r;
  if (logits) {
    err = hipMemcpyAsync(logits, e->logits, sizeof(float) * e->lay.V, hipMemcpyDeviceToHost,
                         e->stream);
    if (err != hipSuccess) return rc(err);
  }
  err = hipMemcpyAsync(e->st_host, e->st, sizeof(StepState), hipMemcpyDeviceToHost, e->stream);
  if (err == hipSuccess) err = hipStreamSynchronize(e->stream);
  if (err != hipSuccess) return rc(err);
  const int de = check_device_error(e);
  if (de != KL_OK) return de;
  if (next) *next = e->st_host->sampled;
  return KL_OK;
}

}  // extern "C"

namespace {

// Rows per prefill pass: 4096 (every BASELINE prompt in one pass; a 4000-row
// pass fills Qwen2.5-1.5B's cache 10% faster than 1024-row chunks, the GEMMs
// having four times the tiles per launch), or KL_PREFILL_CHUNK (64 or more,
// read per call).  Scratch grows with it: about 1.4 GB at 4096 rows for
// Llama2-7B's widths.
int prefill_chunk_rows() {
  const char* e = std::getenv("KL_PREFILL_CHUNK");
  const int v = e ? std::atoi(e) : 4096;
  return v >= 64 ? v : 4096;
}
constexpr int kPrefillMaxSplits = 4;

constexpr int kPrefillMaxSplitsQ8 = 16;  // int8 weights, at most 32 rows

// Split-K factor for a GEMM launch of rows x n outputs (all of its outputs
// together) over k.  fp32 weights / int8 over 32 rows: enough 64 x 64
// workgroup tiles to fill the chip, each split keeping >= 32 k blocks.
// int8 with at most 32 rows (32 x 128 tiles, one per 128 outputs): the split
// (up to kPrefillMaxSplitsQ8) that minimises rounds of resident workgroups x
// k blocks per split, `slots` workgroups resident at once (5 per CU for the
// direct-to-LDS int8 kernel, 3 for the register-staged one).
int prefill_splits(int rows, int n, int k, bool q8, int slots = 768) {
  int s = 1;
  if (q8 && rows <= 32) {
    const long long tiles = (n + 127) / 128, nkb = k / 32;
    long long best = -1;
    for (int t = 1; t <= kPrefillMaxSplitsQ8 && t <= nkb; ++t) {
      const long long cost = (tiles * t + slots - 1) / slots * ((nkb + t - 1) / t);
      if (best < 0 || cost < best) {
        best = cost;
        s = t;
      }
    }
    return s;
  }
  const long long tiles = static_cast<long long>((rows + 63) / 64) * ((n + 63) / 64);
  while (s < kPrefillMaxSplits && tiles * s < 1024 && k / 16 / (2 * s) >= 32) s *= 2;
  return s;
}

bool prefill_supported(const kl_engine* e) {
  const ImageLayout& m = e->lay;
  const int hd = m.hd;
  if (hd != 32 && hd != 64 && hd != 128 && hd != 256) return false;
  // int8 GEMMs take whole 32-column blocks and groups of at least 4.
  if (e->quant && (m.D % kGemmBK || m.Dq % kGemmBK || m.F % kGemmBK || m.gs < 4 ||
                   (m.gs & (m.gs - 1))))
    return false;
  return true;
}

// One projection of a layer as a GEMM segment (fp32 or int8 weights, dense
// rows of K columns).
GemmSeg proj_seg(const kl_engine* e, const WView& w, float* C, const float* bias, int N, int K,
                 int ldc) {
  GemmSeg sg{};
  sg.W = w.w;
  sg.C = C;
  sg.bias = bias;
  sg.N = N;
  sg.ldw = K;
  sg.ldc = ldc;
  if (e->quant) {
    sg.S = w.s;
    while ((1 << sg.gshift) < e->lay.gs) ++sg.gshift;
  }
  return sg;
}

// Allocates the prefill scratch for `rows` rows (once; grows if needed).
int prefill_scratch(kl_engine* e, int rows) {
  if (rows <= e->pf_rows) return KL_OK;
  const ImageLayout& m = e->lay;
  size_t am = 0;
  int r = kl_argmax_workspace_size(m.V, &am);
  if (r != KL_OK) return r;
  auto al = [](size_t b) { return (b + 255) & ~size_t(255); };
  const size_t R = rows;
  const size_t sz_x = al(R * m.D * 4), sz_q = al(R * m.Dq * 4), sz_h = al(R * m.F * 4);
  size_t attn_ws = 0;
  r = kl_attn_prefill_workspace_size(rows, m.H, m.hd, &attn_ws);
  if (r != KL_OK) return r;
  // Split-K partials: up to kPrefillMaxSplits x rows x D (the WO and W2
  // outputs), and for int8 prompts of at most 32 rows also the grouped QKV
  // and W1/W3 outputs at up to kPrefillMaxSplitsQ8 splits.
  size_t ws_floats = static_cast<size_t>(kPrefillMaxSplits) * R * m.D;
  // The split-product GEMMs choose up to 8 splits for WO and W2, 4 for the
  // grouped q/k/v and 2 for W1/W3 within this workspace.
  if (e->pf_x6)
    ws_floats = std::max({ws_floats, 8 * R * m.D, 4 * R * (static_cast<size_t>(m.Dq) + 2 * m.Dkv),
                          2 * R * 2 * static_cast<size_t>(m.F)});
  if (e->quant)
    ws_floats = std::max(ws_floats, static_cast<size_t>(kPrefillMaxSplitsQ8) * std::min<size_t>(R, 32) *
                                        std::max<size_t>({static_cast<size_t>(m.Dq) + 2 * m.Dkv,
                                                          2 * static_cast<size_t>(m.F),
                                                          static_cast<size_t>(m.D)}));
  const size_t sz_ws = al(ws_floats * 4);
  const int kmax = std::max({m.D, m.Dq, m.F});
  const size_t sz_ax = e->pf_x6 ? al(x6_plane_bytes(rows, kmax)) : e->pf_q8s ? al(q8s_aplane_bytes(kmax)) : 0;
  const size_t total = 2 * sz_x + 2 * sz_q + 2 * sz_h + sz_ws + al(attn_ws) + al(m.D * 4) +
                       al(m.S * 4) + al(256) + al(am) + sz_ax;
  char* buf = nullptr;
  hipError_t err = hipMalloc(&buf, total);
  if (err != hipSuccess) return KL_ENOMEM;
  if (e->pf_buf) (void)hipFree(e->pf_buf);
  e->pf_buf = buf;
  size_t off = 0;
  auto take = [&](size_t b) {
    char* p = buf + off;
    off += b;
    return p;
  };
  e->pf_x = reinterpret_cast<float*>(take(sz_x));
  e->pf_xn = reinterpret_cast<float*>(take(sz_x));
  e->pf_q = reinterpret_cast<float*>(take(sz_q));
  e->pf_att = reinterpret_cast<float*>(take(sz_q));
  e->pf_h1 = reinterpret_cast<float*>(take(sz_h));
  e->pf_h3 = reinterpret_cast<float*>(take(sz_h));
  e->pf_ws = reinterpret_cast<float*>(take(sz_ws));
  e->pf_ws_bytes = sz_ws;
  e->pf_aws = take(al(attn_ws));
  e->pf_aws_bytes = attn_ws;
  e->pf_xlast = reinterpret_cast<float*>(take(al(m.D * 4)));
  e->pf_tok = reinterpret_cast<int32_t*>(take(al(m.S * 4)));
  e->pf_next = reinterpret_cast<int32_t*>(take(al(256)));
  e->pf_am = take(al(am));
  e->pf_am_bytes = am;
  e->pf_ax = sz_ax ? take(sz_ax) : nullptr;
  e->pf_rows = rows;
  err = hipMemsetAsync(e->pf_am, 0, am, e->stream);
  if (err != hipSuccess) return rc(err);
  return KL_OK;
}

// Builds the bf16 planes of every layer's fp32 projections, or the packed
// int8 projections where a chunk of `last_rows` (<= 32) rows will use them
// (once).
int prefill_planes(kl_engine* e, int last_rows) {
  if (e->xw_buf) return KL_OK;
  const ImageLayout& m = e->lay;
  if (e->pf_q8s && last_rows <= 32) {
    const int D = m.D, Dq = m.Dq, Dkv = m.Dkv, F = m.F, gs = m.gs;
    auto pb = [&](int N, int K) { return (q8s_packed_bytes(N, K, gs) + 255) & ~size_t(255); };
    const size_t per_layer = pb(Dq, D) + 2 * pb(Dkv, D) + pb(D, Dq) + 2 * pb(F, D) + pb(D, F);
    char* buf = nullptr;
    if (hipMalloc(&buf, per_layer * m.L) != hipSuccess) return KL_ENOMEM;
    e->xw_buf = buf;
    hipStream_t hs = static_cast<hipStream_t>(e->stream);
    size_t off = 0;
    int r = KL_OK;
    auto pack = [&](const WView& w, int N, int K) -> const void* {
      char* dst = buf + off;
      off += (q8s_packed_bytes(N, K, gs) + 255) & ~size_t(255);
      if (r == KL_OK) r = q8s_pack_run(static_cast<const int8_t*>(w.w), w.s, N, K, gs, dst, hs);
      return dst;
    };
    for (int l = 0; l < m.L; ++l) {
      LayerDev& Ld = e->layers[l];
      Ld.xp.q = pack(Ld.wq, Dq, D);
      Ld.xp.k = pack(Ld.wk, Dkv, D);
      Ld.xp.v = pack(Ld.wv, Dkv, D);
      Ld.xp.o = pack(Ld.wo, D, Dq);
      Ld.xp.w1 = pack(Ld.w1, F, D);
      Ld.xp.w2 = pack(Ld.w2, D, F);
      Ld.xp.w3 = pack(Ld.w3, F, D);
    }
    return r;
  }
  if (!e->pf_x6) return KL_OK;
  const int D = m.D, Dq = m.Dq, Dkv = m.Dkv, F = m.F;
  const size_t per_layer = x6_plane_bytes(Dq, D) + 2 * x6_plane_bytes(Dkv, D) + x6_plane_bytes(D, Dq) +
                           2 * x6_plane_bytes(F, D) + x6_plane_bytes(D, F);
  char* buf = nullptr;
  hipError_t err = hipMalloc(&buf, per_layer * m.L);
  if (err != hipSuccess) return KL_ENOMEM;
  e->xw_buf = buf;
  hipStream_t hs = static_cast<hipStream_t>(e->stream);
  size_t off = 0;
  int r = KL_OK;
  auto planes = [&](const WView& w, int N, int K) -> const void* {
    char* dst = buf + off;
    off += x6_plane_bytes(N, K);
    if (r == KL_OK) r = split3_run(static_cast<const float*>(w.w), N, K, K, dst, hs);
    return dst;
  };
  for (int l = 0; l < m.L; ++l) {
    LayerDev& Ld = e->layers[l];
    Ld.xp.q = planes(Ld.wq, Dq, D);
    Ld.xp.k = planes(Ld.wk, Dkv, D);
    Ld.xp.v = planes(Ld.wv, Dkv, D);
    Ld.xp.o = planes(Ld.wo, D, Dq);
    Ld.xp.w1 = planes(Ld.w1, F, D);
    Ld.xp.w2 = planes(Ld.w2, D, F);
    Ld.xp.w3 = planes(Ld.w3, F, D);
    Ld.xp.one = 0;
  }
  // Which matrices are bf16-exact (planes 1 and 2 all zero): one flag word per
  // matrix, read back once.
  if (r != KL_OK) return r;
  unsigned* flags = nullptr;
  const size_t nf = 7 * static_cast<size_t>(m.L);
  if (hipMalloc(&flags, nf * sizeof(unsigned)) != hipSuccess) return KL_ENOMEM;
  r = rc(hipMemsetAsync(flags, 0, nf * sizeof(unsigned), hs));
  for (int l = 0; l < m.L && r == KL_OK; ++l) {
    const XPlanes& xp = e->layers[l].xp;
    const void* pl[7] = {xp.q, xp.k, xp.v, xp.o, xp.w1, xp.w2, xp.w3};
    const int rows[7] = {Dq, Dkv, Dkv, D, F, D, F}, cols[7] = {D, D, D, Dq, D, F, D};
    for (int i = 0; i < 7 && r == KL_OK; ++i)
      r = x6_planes_flag_run(pl[i], rows[i], cols[i], flags + 7 * l + i, hs);
  }
  std::vector<unsigned> h(nf, 1u);
  if (r == KL_OK) r = rc(hipMemcpyAsync(h.data(), flags, nf * sizeof(unsigned), hipMemcpyDeviceToHost, hs));
  if (r == KL_OK) r = rc(hipStreamSynchronize(hs));
  (void)hipFree(flags);
  for (int l = 0; l < m.L && r == KL_OK; ++l)
    for (int i = 0; i < 7; ++i)
      if (h[7 * l + i] == 0) e->layers[l].xp.one |= 1u << i;
  return r;
}

// Positions pos0 .. pos0+n-1 through every layer; leaves the residual rows in
// pf_x and the K/V rows in the caches.
int prefill_chunk(kl_engine* e, int pos0, int n) {
  const ImageLayout& m = e->lay;
  const int D = m.D, Dq = m.Dq, Dkv = m.Dkv, F = m.F, H = m.H, KVH = m.KVH, hd = m.hd;
  const bool q8 = e->quant != 0;
  void* st = e->stream;
  hipStream_t hs = static_cast<hipStream_t>(st);
  const size_t kv_layer = static_cast<size_t>(m.S) * Dkv;
  int r = kl_embedding(e->pf_tok + pos0, n, e->emb, m.V, D, e->pf_x, nullptr, st);
#define PF(call)          \
  do {                    \
    if (r == KL_OK) r = (call); \
  } while (0)
  // fp32 weights: split-product GEMMs over bf16 planes of the weights
  // (prefill_planes) and of each GEMM input; int8 weights with at most 32
  // rows: k_gemm_q8s over the packed weights.  On these paths every GEMM
  // input is written as planes by its producer (the row norms, SwiGLU, or a
  // split of the attention output), and the split-K partials of Wo, W1/W3
  // and W2 are summed by the next producer instead of a reduction pass
  // (pend: W2's partials of the previous layer, not yet added to pf_x).
  const bool q8s = e->pf_q8s && n <= 32 && e->xw_buf;
  const bool fast = e->pf_x6 || q8s;
  const size_t nD = static_cast<size_t>(n) * D, nF = static_cast<size_t>(n) * F;
  int pend = 0;
  // wone: every W of the launch is bf16-exact (plane 0 only).
  auto gemm_fast = [&](int k, int nseg, const GemmSeg* sg, const void* const* wx, int acc, int* deferred,
                       bool wone) {
    if (q8s) {
      GemmSeg s2[kGemmMaxSeg];
      for (int i = 0; i < nseg; ++i) {
        s2[i] = sg[i];
        s2[i].W = wx[i];
      }
      PF(gemm_run_q8s(e->pf_ax, n, k, m.gs, nseg, s2, acc, e->pf_ws, e->pf_ws_bytes, hs, deferred));
      return;
    }
    GemmX6Planes p{};
    p.A = e->pf_ax;
    for (int i = 0; i < nseg; ++i) p.W[i] = wx[i];
    p.w_planes = wone ? 1 : 3;
    PF(gemm_run_x6(p, n, k, nseg, sg, acc, e->pf_ws, e->pf_ws_bytes, hs, deferred));
  };
  for (int l = 0; l < m.L && r == KL_OK; ++l) {
    const LayerDev& Ld = e->layers[l];
    float* kc = e->kcache + l * kv_layer;
    float* vc = e->vcache + l * kv_layer;
    float* krow = kc + static_cast<size_t>(pos0) * Dkv;
    float* vrow = vc + static_cast<size_t>(pos0) * Dkv;
    int dqkv = 1;  // Q/K/V splits left unsummed
    // Split-K where the launch would leave CUs idle (int8, at most 32 rows);
    // every split's partials fit pf_ws (prefill_scratch).  Groups of at least
    // 32 run the direct-to-LDS int8 kernel (5 workgroups per CU).
    const int slots = (m.gs >= 32 ? 5 : 3) * 256;
    auto splits_for = [&](int ntot, int k, bool grouped) {
      const int sp = grouped && !(q8 && n <= 32) ? 1 : prefill_splits(n, ntot, k, q8, slots);
      if (r == KL_OK && sp > 1 && static_cast<size_t>(sp) * n * ntot * sizeof(float) > e->pf_ws_bytes)
        r = KL_EWORKSPACE;
      return sp;
    };
    // attention_rms + attention_qkv (llama3.cpp:599-639; qwen3.cpp:470-513):
    // q, k and v in one grouped launch (k and v straight into the cache rows)
    {
      const GemmSeg sg[3] = {proj_seg(e, Ld.wq, e->pf_q, Ld.bq, Dq, D, Dq),
                             proj_seg(e, Ld.wk, krow, Ld.bk, Dkv, D, Dkv),
                             proj_seg(e, Ld.wv, vrow, Ld.bv, Dkv, D, Dkv)};
      if (fast) {
        PF(norm_planes_run(e->pf_x, Ld.rms_att, n, D, e->eps, e->pf_ws, pend, nD, e->pf_ax, q8s, hs));
        pend = 0;
        const void* wx[3] = {Ld.xp.q, Ld.xp.k, Ld.xp.v};
        // Short int8 prompts leave Q/K/V's split-K partials to the rotation
        // (one pass summing and rotating them); Qwen3's q/k norm needs the sums first.
        gemm_fast(D, 3, sg, wx, 0, q8s && e->transform != 2 ? &dqkv : nullptr, (Ld.xp.one & 7u) == 7u);
      } else {
        PF(kl_rmsnorm_rows(e->pf_x, Ld.rms_att, e->pf_xn, n, D, e->eps, st));
        const int sp = splits_for(Dq + 2 * Dkv, D, true);
        PF(gemm_run(e->pf_xn, n, D, D, 3, sg, 0, e->pf_ws, sp, hs));
      }
    }
    if (e->transform == 2 && (hd == 64 || hd == 128)) {  // Qwen3 q/k RMSNorm (eps 1e-6) + RoPE
      PF(kl_qk_norm_rope_rows(e->rope_style, hd, H, KVH, e->pf_q, Dq, krow, Dkv, Ld.qn, Ld.kn, 1e-6f,
                              pos0, n, e->sin_t, e->cos_t, st));
    } else {
      if (e->transform == 2) {
        PF(kl_rmsnorm_rows(e->pf_q, Ld.qn, e->pf_q, n * H, hd, 1e-6f, st));
        PF(kl_rmsnorm_rows(krow, Ld.kn, krow, n * KVH, hd, 1e-6f, st));
      }
      if (dqkv > 1)
        PF(qkv_sum_rope_run(e->rope_style, Dq, Dkv, hd, e->pf_ws, dqkv,
                            static_cast<size_t>(n) * (Dq + 2 * static_cast<size_t>(Dkv)), Ld.bq, Ld.bk, Ld.bv,
                            e->pf_q, Dq, krow, Dkv, vrow, Dkv, pos0, n, e->sin_t, e->cos_t, hs));
      else
        PF(kl_rope_rows(e->rope_style, Dq, Dkv, hd, e->pf_q, Dq, krow, Dkv, pos0, n, e->sin_t,
                        e->cos_t, st));
    }
    // attention_mha (llama3.cpp:651-669), then x += Wo . att
    PF(kl_attn_prefill_ws(pos0, n, H, H / KVH, hd, e->pf_q, Dq, kc, vc, Dkv, e->pf_att, Dq,
                          e->pf_aws, e->pf_aws_bytes, st));
    // feed_forward (llama3.cpp:671-719)
    if (fast) {
      int dwo = 1, d13 = 1, d2 = 1;
      const GemmSeg so = proj_seg(e, Ld.wo, e->pf_x, nullptr, D, Dq, D);
      PF(q8s ? q8s_split_run(e->pf_att, n, Dq, Dq, e->pf_ax, hs) : split3_run(e->pf_att, n, Dq, Dq, e->pf_ax, hs));
      gemm_fast(Dq, 1, &so, &Ld.xp.o, 1, &dwo, (Ld.xp.one >> 3) & 1u);
      PF(norm_planes_run(e->pf_x, Ld.rms_ffn, n, D, e->eps, e->pf_ws, dwo > 1 ? dwo : 0, nD, e->pf_ax,
                         q8s, hs));
      const GemmSeg s13[2] = {proj_seg(e, Ld.w1, e->pf_h1, nullptr, F, D, F),
                              proj_seg(e, Ld.w3, e->pf_h3, nullptr, F, D, F)};
      const void* wx[2] = {Ld.xp.w1, Ld.xp.w3};
      gemm_fast(D, 2, s13, wx, 0, &d13, (Ld.xp.one & 0x50u) == 0x50u);
      PF(swiglu_planes_run(e->pf_h1, e->pf_h3, n, F, e->pf_ws, d13 > 1 ? d13 : 0, 2 * nF, nF, e->pf_ax,
                           q8s, hs));
      const GemmSeg s2 = proj_seg(e, Ld.w2, e->pf_x, nullptr, D, F, D);
      gemm_fast(F, 1, &s2, &Ld.xp.w2, 1, &d2, (Ld.xp.one >> 5) & 1u);
      pend = d2 > 1 ? d2 : 0;
    } else {
      {
        const GemmSeg sg = proj_seg(e, Ld.wo, e->pf_x, nullptr, D, Dq, D);
        const int sp = splits_for(D, Dq, false);
        PF(gemm_run(e->pf_att, n, Dq, Dq, 1, &sg, 1, e->pf_ws, sp, hs));
      }
      PF(kl_rmsnorm_rows(e->pf_x, Ld.rms_ffn, e->pf_xn, n, D, e->eps, st));
      {
        const GemmSeg sg[2] = {proj_seg(e, Ld.w1, e->pf_h1, nullptr, F, D, F),
                               proj_seg(e, Ld.w3, e->pf_h3, nullptr, F, D, F)};
        const int sp = splits_for(2 * F, D, true);
        PF(gemm_run(e->pf_xn, n, D, D, 2, sg, 0, e->pf_ws, sp, hs));
      }
      PF(kl_swiglu(e->pf_h1, e->pf_h3, e->pf_h1, n * F, st));
      {
        const GemmSeg sg = proj_seg(e, Ld.w2, e->pf_x, nullptr, D, F, D);
        const int sp = splits_for(D, F, false);
        PF(gemm_run(e->pf_h1, n, F, F, 1, &sg, 1, e->pf_ws, sp, hs));
      }
    }
  }
  if (pend) PF(partials_add_run(e->pf_x, n, D, e->pf_ws, pend, hs));  // the last layer's W2
#undef PF
  return r;
}

}  // namespace

extern "C" {

int kl_engine_set_prefill(kl_engine* e, int enable) {
  if (!e) return KL_EINVAL;
  if (enable && !prefill_supported(e)) return KL_EUNSUPP;
  e->use_prefill = enable != 0;
  return KL_OK;
}

int kl_engine_prefill(kl_engine* e, const int32_t* prompt, int P, int32_t* next, float* logits,
                      float* prefill_ms) {
  if (!e || !prompt || P <= 0) return KL_EINVAL;
  const ImageLayout& m = e->lay;
  if (P > m.S) return KL_EINVAL;
  for (int i = 0; i < P; ++i)
    if (prompt[i] < 0 || prompt[i] >= m.V) return KL_ETOKEN;
  if (!prefill_supported(e)) return KL_EUNSUPP;
  const int chunk = prefill_chunk_rows();
  int r = prefill_scratch(e, std::min(P, chunk));
  if (r == KL_OK) r = prefill_planes(e, (P - 1) % chunk + 1);
  if (r != KL_OK) return r;
  hipError_t err = hipMemcpyAsync(e->pf_tok, prompt, sizeof(int32_t) * P, hipMemcpyHostToDevice,
                                  e->stream);
  if (err == hipSuccess) err = hipEventRecord(e->ev0, e->stream);
  if (err != hipSuccess) return rc(err);
  int last_n = 0;
  for (int pos0 = 0; pos0 < P && r == KL_OK; pos0 += chunk) {
    last_n = std::min(chunk, P - pos0);
    r = prefill_chunk(e, pos0, last_n);
  }
  // cls_logits + post_processing of position P-1 (llama3.cpp:721-744)
  if (r == KL_OK)
    r = kl_rmsnorm(e->pf_x + static_cast<size_t>(last_n - 1) * m.D, e->rms_final, e->pf_xlast, m.D,
                   e->eps, e->stream);
  if (r == KL_OK)
    r = e->quant ? kl_gemv_q8(e->pf_xlast, static_cast<const int8_t*>(e->wcls.w), e->wcls.s,
                              e->logits, m.V, m.D, m.gs, e->stream)
                 : kl_gemv_f32(e->pf_xlast, static_cast<const float*>(e->wcls.w), e->logits, m.V,
                               m.D, 1.f, e->stream);
  if (r == KL_OK) r = kl_argmax(e->logits, m.V, e->pf_next, e->pf_am, e->pf_am_bytes, e->stream);
  if (r != KL_OK) return r;
  err = hipEventRecord(e->ev1, e->stream);
  int32_t nx = -1;
  if (err == hipSuccess)
    err = hipMemcpyAsync(&nx, e->pf_next, sizeof(int32_t), hipMemcpyDeviceToHost, e->stream);
  if (err == hipSuccess && logits)
    err = hipMemcpyAsync(logits, e->logits, sizeof(float) * m.V, hipMemcpyDeviceToHost, e->stream);
  if (err == hipSuccess) err = hipStreamSynchronize(e->stream);
  if (err == hipSuccess && prefill_ms) err = hipEventElapsedTime(prefill_ms, e->ev0, e->ev1);
  if (err != hipSuccess) return rc(err);
  if (next) *next = nx;
  return KL_OK;
}

int kl_engine_generate(kl_engine* e, const int32_t* prompt, int P, int n_new, int32_t* out_tokens,
                       float* decode_ms) {
  if (!e || !prompt || !out_tokens || P <= 0 || n_new <= 0) return KL_EINVAL;
  if (P + n_new - 1 > e->lay.S) return KL_EINVAL;
  for (int i = 0; i < P; ++i)
    if (prompt[i] < 0 || prompt[i] >= e->lay.V) return KL_ETOKEN;
  if (e->use_prefill && P >= 2) {
    // The prompt in one batched pass; its token is the first of out_tokens,
    // the device loop continues at position P.
    int32_t first = -1;
    int r = kl_engine_prefill(e, prompt, P, &first, nullptr, nullptr);
    if (r != KL_OK) return r;
    out_tokens[0] = first;
    if (decode_ms) *decode_ms = 0.f;
    if (n_new == 1) return KL_OK;
    hipError_t err = set_state(e, StepState{P, first, P, first});
    if (err == hipSuccess) err = hipEventRecord(e->ev0, e->stream);
    if (err != hipSuccess) return rc(err);
    for (int i = 0; i < n_new - 1; ++i) {
      r = run_step(e);
      if (r != KL_OK) return r;
    }
    err = hipEventRecord(e->ev1, e->stream);
    if (err == hipSuccess)
      err = hipMemcpyAsync(out_tokens + 1, e->out_tokens + P, sizeof(int32_t) * (n_new - 1),
                           hipMemcpyDeviceToHost, e->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(e->stream);
    if (err != hipSuccess) return rc(err);
    const int de = check_device_error(e);
    if (de != KL_OK) return de;
    if (decode_ms) {
      err = hipEventElapsedTime(decode_ms, e->ev0, e->ev1);
      if (err != hipSuccess) return rc(err);
    }
    return KL_OK;
  }
  hipError_t err = hipMemcpyAsync(e->prompt, prompt, sizeof(int32_t) * P, hipMemcpyHostToDevice,
                                  e->stream);
  if (err != hipSuccess) return rc(err);
  err = set_state(e, StepState{0, prompt[0], P, 0});
  if (err != hipSuccess) return rc(err);
  // Prompt positions 0 .. P-2, then n_new sampled positions P-1 .. P+n_new-2.
  for (int i = 0; i < P - 1; ++i) {
    const int r = run_step(e);
    if (r != KL_OK) return r;
  }
  err = hipEventRecord(e->ev0, e->stream);
  if (err != hipSuccess) return rc(err);
  for (int i = 0; i < n_new; ++i) {
    const int r = run_step(e);
    if (r != KL_OK) return r;
  }
  err = hipEventRecord(e->ev1, e->stream);
  if (err == hipSuccess)
    err = hipMemcpyAsync(out_tokens, e->out_tokens + (P - 1), sizeof(int32_t) * n_new,
                         hipMemcpyDeviceToHost, e->stream);
  if (err == hipSuccess) err = hipStreamSynchronize(e->stream);
  if (err != hipSuccess) return rc(err);
  const int de = check_device_error(e);
  if (de != KL_OK) return de;
  if (decode_ms) {
    err = hipEventElapsedTime(decode_ms, e->ev0, e->ev1);
    if (err != hipSuccess) return rc(err);
  }
  return KL_OK;
}

int kl_engine_bench(kl_engine* e, const int32_t* prompt, int P, int n_warmup, int n_timed,
                    int32_t* out_tokens, float* timed_ms) {
  if (!e || !prompt || !out_tokens || !timed_ms || P <= 0 || n_warmup < 0 || n_timed <= 0)
    return KL_EINVAL;
  if (P + n_warmup + n_timed - 1 > e->lay.S) return KL_EINVAL;
  for (int i = 0; i < P; ++i)
    if (prompt[i] < 0 || prompt[i] >= e->lay.V) return KL_ETOKEN;
  // With the batched prefill on, the prompt (positions 0 .. P-1, the first
  // warm-up step included) is one kl_engine_prefill call; the timed steps
  // run at the same positions either way.
  const bool batched = e->use_prefill && P >= 2 && n_warmup >= 1;
  int32_t first = -1;
  hipError_t err = hipSuccess;
  if (batched) {
    int r = kl_engine_prefill(e, prompt, P, &first, nullptr, nullptr);
    if (r != KL_OK) return r;
    err = set_state(e, StepState{P, first, P, first});
    if (err != hipSuccess) return rc(err);
    for (int i = 0; i < n_warmup - 1; ++i) {
      r = run_step(e);
      if (r != KL_OK) return r;
    }
  } else {
    err = hipMemcpyAsync(e->prompt, prompt, sizeof(int32_t) * P, hipMemcpyHostToDevice, e->stream);
    if (err != hipSuccess) return rc(err);
    err = set_state(e, StepState{0, prompt[0], P, 0});
    if (err != hipSuccess) return rc(err);
    for (int i = 0; i < P - 1 + n_warmup; ++i) {
      const int r = run_step(e);
      if (r != KL_OK) return r;
    }
  }
  err = hipStreamSynchronize(e->stream);
  if (err == hipSuccess) err = hipEventRecord(e->ev0, e->stream);
  if (err != hipSuccess) return rc(err);
  for (int i = 0; i < n_timed; ++i) {
    const int r = run_step(e);
    if (r != KL_OK) return r;
  }
  err = hipEventRecord(e->ev1, e->stream);
  if (err == hipSuccess) err = hipStreamSynchronize(e->stream);
  if (err == hipSuccess) err = hipEventElapsedTime(timed_ms, e->ev0, e->ev1);
  if (err == hipSuccess && batched) {
    out_tokens[0] = first;  // sampled by the prefill at position P-1
    err = hipMemcpy(out_tokens + 1, e->out_tokens + P, sizeof(int32_t) * (n_warmup + n_timed - 1),
                    hipMemcpyDeviceToHost);
  } else if (err == hipSuccess) {
    err = hipMemcpy(out_tokens, e->out_tokens + (P - 1), sizeof(int32_t) * (n_warmup + n_timed),
                    hipMemcpyDeviceToHost);
  }
  if (err != hipSuccess) return rc(err);
  return check_device_error(e);
}

int kl_engine_trace_step(kl_engine* e, int32_t token, int32_t pos, uint64_t* ticks,
                         int64_t max_ticks, int32_t* n_slots, int32_t* n_workgroups) {
  if (!e || !n_slots || !n_workgroups) return KL_EINVAL;
  if (e->mode != KL_MODE_PERSISTENT) return KL_EUNSUPP;
  if (pos < 0 || pos >= e->lay.S) return KL_EINVAL;
  if (token < 0 || token >= e->lay.V) return KL_ETOKEN;
  const int slots = 2 * 5 * e->lay.L + 3;
  const size_t n = static_cast<size_t>(slots) * e->nwg;
  *n_slots = slots;
  *n_workgroups = e->nwg;
  if (!ticks || static_cast<int64_t>(n) > max_ticks) return KL_EWORKSPACE;
  return trace_once(e, token, pos, reinterpret_cast<unsigned long long*>(ticks));
}

int kl_engine_profile(kl_engine* e, int32_t token, int32_t pos0, int steps, float* avg_ms,
                      int32_t* counts) {
  if (!e || !avg_ms || !counts || steps <= 0) return KL_EINVAL;
  if (pos0 < 0 || pos0 + steps > e->lay.S) return KL_EINVAL;
  if (token < 0 || token >= e->lay.V) return KL_ETOKEN;
  for (int k = 0; k < kKinds; ++k) {
    avg_ms[k] = 0.f;
    counts[k] = 0;
  }
  hipError_t err = set_state(e, StepState{pos0, token, 0, 0});
  if (err != hipSuccess) return rc(err);
  std::vector<hipEvent_t> ev;
  std::vector<int> kinds;
  Marks mk{&ev, &kinds};
  int r = KL_OK;
  const bool pers = e->mode == KL_MODE_PERSISTENT;
  for (int i = 0; i < steps && r == KL_OK; ++i)
    r = pers ? launch_persistent(e, &mk) : launch_step(e, &mk);
  err = hipStreamSynchronize(e->stream);
  if (r == KL_OK && err != hipSuccess) r = rc(err);
  if (r == KL_OK) r = check_device_error(e);
  for (size_t i = 0; r == KL_OK && i + 1 < ev.size(); ++i) {
    if (kinds[i] == kKEnd) continue;  // end-of-step mark
    float ms = 0.f;
    err = hipEventElapsedTime(&ms, ev[i], ev[i + 1]);
    if (err != hipSuccess) {
      r = rc(err);
      break;
    }
    avg_ms[kinds[i]] += ms;
    counts[kinds[i]] += 1;
  }
  for (hipEvent_t x : ev) (void)hipEventDestroy(x);
  if (r != KL_OK) return r;
  for (int k = 0; k < kKinds; ++k)
    if (counts[k]) avg_ms[k] /= static_cast<float>(counts[k]);
  return KL_OK;
}

int kl_engine_buffers(const kl_engine* e, const float** logits, const float** key_cache,
                      const float** value_cache) {
  if (!e) return KL_EINVAL;
  if (logits) *logits = e->logits;
  if (key_cache) *key_cache = e->kcache;
  if (value_cache) *value_cache = e->vcache;
  return KL_OK;
}

int kl_engine_stream(const kl_engine* e, void** stream) {
  if (!e || !stream) return KL_EINVAL;
  *stream = e->stream;
  return KL_OK;
}

}  // extern "C"
