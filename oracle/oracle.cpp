// CPU parity oracle for the KuiperLLama batch-1 decode path.
//
// TEST INFRASTRUCTURE ONLY -- see oracle.h.  Built with g++ -O3
// -ffp-contract=off (no fused multiply-add anywhere, so elementwise results
// such as RoPE and int8 dequant are reproducible bit-for-bit), OpenMP over
// independent rows/heads (each output element is still produced by one thread
// in one fixed order, so results do not depend on the thread count).
#include "oracle.h"

#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

namespace {

// Fixed-order fp32 dot product: 8 interleaved accumulators (lane c % 8),
// folded pairwise, then the scalar tail.  The reference delegates this to
// OpenBLAS sgemv through Armadillo (kernels/cpu/matmul_kernel.cpp:37-40),
// whose internal order is not reproducible here; this order is the oracle's
// own documented choice.
inline float dot8(const float* a, const float* b, int n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int c = 0;
  for (; c + 8 <= n; c += 8) {
    for (int k = 0; k < 8; ++k) acc[k] += a[c + k] * b[c + k];
  }
  float s = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
  for (; c < n; ++c) s += a[c] * b[c];
  return s;
}

// Armadillo's arrayops::accumulate order: two interleaved accumulators (even
// and odd indices), summed at the end.  Used by arma::mean / arma::sum, i.e.
// the CPU RMSNorm mean (kernels/cpu/rmsnorm_kernel.cpp:30) and the softmax sum
// (kernels/cpu/softmax_kernel.cpp:13).
inline float arma_accumulate(const float* x, int n) {
  float acc1 = 0.f, acc2 = 0.f;
  int i = 0, j = 1;
  for (; j < n; i += 2, j += 2) {
    acc1 += x[i];
    acc2 += x[j];
  }
  if (i < n) acc1 += x[i];
  return acc1 + acc2;
}

typedef float ov8 __attribute__((vector_size(32)));
typedef int8_t oq8 __attribute__((vector_size(8)));

inline ov8 ld8(const float* p) {
  ov8 v;
  std::memcpy(&v, p, sizeof(v));
  return v;
}

inline float fold8(const ov8 a) {
  return ((a[0] + a[4]) + (a[1] + a[5])) + ((a[2] + a[6]) + (a[3] + a[7]));
}

// The int8 counterpart of q8_row_dot for RB rows x TB positions.  Needs
// group_size % 8 == 0 and cols % 8 == 0, so that the 8 columns of a step
// share one scale: each lane still forms (x * scale) * float(q).
template <int RB, int TB>
void tile_q8(const int8_t* Q, const float* S, int64_t row0, int cols, int gs, const float* X,
             int64_t ldx, float* Y, int64_t ldy) {
  ov8 acc[RB][TB];
  for (int j = 0; j < RB; ++j)
    for (int i = 0; i < TB; ++i) acc[j][i] = ov8{0, 0, 0, 0, 0, 0, 0, 0};
  for (int c = 0; c < cols; c += 8) {
    ov8 x[TB];
    for (int i = 0; i < TB; ++i) x[i] = ld8(X + i * ldx + c);
    for (int j = 0; j < RB; ++j) {
      const int64_t base = (row0 + j) * cols + c;
      oq8 qv;
      std::memcpy(&qv, Q + base, sizeof(qv));
      const ov8 qf = __builtin_convertvector(qv, ov8);
      const float sc = S[base / gs];
      for (int i = 0; i < TB; ++i) acc[j][i] += (x[i] * sc) * qf;
    }
  }
  for (int j = 0; j < RB; ++j)
    for (int i = 0; i < TB; ++i) Y[i * ldy + j] = fold8(acc[j][i]);
}

// One row of the int8 GEMV below: 8 interleaved accumulators of
// (x[c] * scale) * float(q), folded as in dot8, then the scalar tail.
inline float q8_row_dot(const float* x, const int8_t* q, const float* scales, int64_t base,
                        int cols, int group_size) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int c = 0;
  for (; c + 8 <= cols; c += 8) {
    for (int k = 0; k < 8; ++k) {
      const int64_t idx = base + c + k;
      acc[k] += (x[c + k] * scales[idx / group_size]) * static_cast<float>(q[idx]);
    }
  }
  float s = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
  for (; c < cols; ++c) {
    const int64_t idx = base + c;
    s += (x[c] * scales[idx / group_size]) * static_cast<float>(q[idx]);
  }
  return s;
}

}  // namespace

extern "C" {

void or_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int or_get_threads(void) { return omp_get_max_threads(); }

// kernels/cpu/matmul_kernel.cpp:5-41: y[r] = (sum_c x[c] * W[r, c]) * scale,
// W row-major [rows x cols] (Armadillo views it as a cols x rows column-major
// matrix and computes x^T * W^T).
void or_gemv_f32(const float* x, const float* W, float* y, int rows, int cols, float scale) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    y[r] = dot8(W + (int64_t)r * cols, x, cols) * scale;
  }
}

// CUDA-only semantics restated (kernels/cuda/matmul_kernel.cu:56-87; there is
// no CPU int8 kernel, kernels_interfaces.cpp:54-61):
//   y[r] = sum_c (x[c] * scales[(r*cols + c) / group_size]) * float(q[r*cols + c])
// The group index is taken over the flattened matrix, as in the reference.
// Where group_size and cols are multiples of 8, the 8 columns of a step share
// one scale and tile_q8 evaluates the same lanes with vector instructions
// (bitwise equal to q8_row_dot, which or_gemv_q8_scalar keeps for the test
// that pins the two together).
void or_gemv_q8(const float* x, const int8_t* q, const float* scales, float* y, int rows, int cols,
                int group_size) {
  if (group_size % 8 == 0 && cols % 8 == 0) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) tile_q8<1, 1>(q, scales, r, cols, group_size, x, 0, y + r, 0);
    return;
  }
  or_gemv_q8_scalar(x, q, scales, y, rows, cols, group_size);
}

void or_gemv_q8_scalar(const float* x, const int8_t* q, const float* scales, float* y, int rows,
                       int cols, int group_size) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) y[r] = q8_row_dot(x, q, scales, (int64_t)r * cols, cols, group_size);
}

// tools/export_llama.py:49-73 (quantize_q80): per contiguous group of
// group_size values, scale = max|w| / 127 (fp32 divide), q = round-half-even
// (w / scale) as int8.  An all-zero group (scale 0, where torch would produce
// NaN) is defined here as q = 0.
void or_quantize_q8(const float* w, int64_t n, int group_size, int8_t* q, float* scales) {
  const int64_t groups = n / group_size;
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < groups; ++g) {
    const float* wg = w + g * group_size;
    float wmax = 0.f;
    for (int i = 0; i < group_size; ++i) wmax = std::max(wmax, std::fabs(wg[i]));
    const float scale = wmax / 127.0f;
    scales[g] = scale;
    for (int i = 0; i < group_size; ++i) {
      float v = scale == 0.f ? 0.f : std::nearbyint(wg[i] / scale);
      q[g * group_size + i] = static_cast<int8_t>(v);
    }
  }
}

// Dequantized value of the reference int8 layout: float(q) * scale, one fp32
// multiply (kernels/cuda/matmul_kernel.cu:73 evaluates the same product).
void or_dequant_q8(const int8_t* q, const float* scales, int64_t n, int group_size, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = scales[i / group_size] * static_cast<float>(q[i]);
}

// kernels/cpu/rmsnorm_kernel.cpp:4-33:
//   mean = mean(x^2) + eps; rsqrt = 1 / sqrt(mean); y = w % (rsqrt * x)
void or_rmsnorm(const float* x, const float* w, float* y, int n, float eps) {
  std::vector<float> sq(n);
  for (int i = 0; i < n; ++i) sq[i] = x[i] * x[i];
  const float mean = arma_accumulate(sq.data(), n) / static_cast<float>(n) + eps;
  const float rsqrt = 1.f / std::sqrt(mean);
  for (int i = 0; i < n; ++i) y[i] = w[i] * (rsqrt * x[i]);
}

// CUDA-only semantics restated (kernels/cuda/rmsnorm_kernel.cu:8-60, launched
// by rmsnorm_kernel_cu_dim :138-164): the same normalisation applied to each
// row of length n independently, with one weight vector of length n.  The
// reference hard-codes eps = 1e-6 (:148); callers pass it explicitly here.
void or_rmsnorm_rows(const float* x, const float* w, float* y, int rows, int n, float eps) {
  for (int r = 0; r < rows; ++r) or_rmsnorm(x + (int64_t)r * n, w, y + (int64_t)r * n, n, eps);
}

// kernels/cpu/rope_kernel.cpp:4-16 / :44-56 / :84-96 (identical bodies, theta
// 5e5 / 1e6 / 1e4 chosen by build flag):
//   freq = 1 / pow(theta, d / hd); val = pos * freq; table = sinf/cosf(val)
void or_sincos_table(int head_size, int seq_len, float theta, float* sin_cache, float* cos_cache) {
  for (int pos = 0; pos < seq_len; ++pos) {
    for (int d = 0; d < head_size; ++d) {
      const float freq =
          1.0f / std::pow(theta, static_cast<float>(d) / static_cast<float>(head_size));
      const float val = static_cast<float>(pos) * freq;
      sin_cache[pos * head_size + d] = std::sin(val);
      cos_cache[pos * head_size + d] = std::cos(val);
    }
  }
}

// Interleaved style: kernels/cpu/rope_kernel.cpp:98-121 (pairs (i, i+1), table
// index i % hd).  Rotate-half style: :18-42 and :58-82 (pairs (j, j + hd/2)
// within each head, table index 2j).  k is rotated only where the q index is
// below kv_dim.
void or_rope(int style, int dim, int kv_dim, int head_size, float* q, float* k, int pos,
             const float* sin_cache, const float* cos_cache) {
  if (style == OR_ROPE_INTERLEAVED) {
    for (int i = 0; i < dim; i += 2) {
      const int hdim = i % head_size;
      const float fci = sin_cache[pos * head_size + hdim];
      const float fcr = cos_cache[pos * head_size + hdim];
      const int rotn = i < kv_dim ? 2 : 1;
      for (int v = 0; v < rotn; ++v) {
        float* vec = v == 0 ? q : k;
        const float v0 = vec[i];
        const float v1 = vec[i + 1];
        vec[i] = v0 * fcr - v1 * fci;
        vec[i + 1] = v0 * fci + v1 * fcr;
      }
    }
  } else {
    const int half = head_size / 2;
    for (int i = 0; i < dim; i += head_size) {
      for (int j = 0; j < half; ++j) {
        const float fci = sin_cache[pos * head_size + j * 2];
        const float fcr = cos_cache[pos * head_size + j * 2];
        const int rotn = i < kv_dim ? 2 : 1;
        for (int v = 0; v < rotn; ++v) {
          float* vec = v == 0 ? q : k;
          const float v0 = vec[i + j];
          const float v1 = vec[i + j + half];
          vec[i + j] = v0 * fcr - v1 * fci;
          vec[i + j + half] = v0 * fci + v1 * fcr;
        }
      }
    }
  }
}

// kernels/cpu/softmax_kernel.cpp:4-15: subtract the max (std::max_element),
// expf, Armadillo sum, divide.
void or_softmax(float* x, int n) {
  const float mx = *std::max_element(x, x + n);
  for (int i = 0; i < n; ++i) x[i] = std::exp(x[i] - mx);
  const float sum = arma_accumulate(x, n);
  for (int i = 0; i < n; ++i) x[i] = x[i] / sum;
}

}  // extern "C"

namespace {

// One head of or_mha: scores of head h against positions 0..pos of one
// layer's caches, softmax, then the weighted sum of V in increasing t.
inline void mha_head(int pos, int h, int kv_dim, int kv_mul, int head_size, float* oh,
                     const float* qh, float* sh, const float* kcache, const float* vcache) {
  const float scale = 1.f / std::sqrt(static_cast<float>(head_size));
  const int64_t head_off = (int64_t)(h / kv_mul) * head_size;
  for (int t = 0; t <= pos; ++t) {
    const float* kt = kcache + (int64_t)t * kv_dim + head_off;
    sh[t] = dot8(qh, kt, head_size) * scale;
  }
  or_softmax(sh, pos + 1);
  for (int d = 0; d < head_size; ++d) oh[d] = 0.f;
  for (int t = 0; t <= pos; ++t) {
    const float* vt = vcache + (int64_t)t * kv_dim + head_off;
    const float p = sh[t];
    for (int d = 0; d < head_size; ++d) oh[d] += p * vt[d];
  }
}

}  // namespace

extern "C" {

// kernels/cpu/mha_kernel.cpp:5-61 with softmax_kernel.cpp:4-15 and
// scale_sum_kernel.cpp:5-22.  Per head h (kv head h / kv_mul):
//   s_t = (q_h . K_t) * (1/sqrt(hd)), t in [0, pos]; softmax; out_h = sum_t p_t V_t
// accumulated in increasing t.  Caches are [layers][seq_len][kv_dim].
void or_mha(int pos, int head_num, int layer_index, int seq_len, int kv_dim, int kv_mul,
            int head_size, float* out, const float* q, float* score, const float* key_cache,
            const float* value_cache) {
  const int64_t layer_offset = (int64_t)layer_index * seq_len * kv_dim;
#pragma omp parallel for schedule(static)
  for (int h = 0; h < head_num; ++h)
    mha_head(pos, h, kv_dim, kv_mul, head_size, out + (int64_t)h * head_size,
             q + (int64_t)h * head_size, score + (int64_t)h * seq_len, key_cache + layer_offset,
             value_cache + layer_offset);
}

// kernels/cpu/scale_kernel.cpp:3-9: x = x * scale (Armadillo's vector times
// scalar: one rounding per element).
void or_scale(float scale, float* x, int n) {
  for (int i = 0; i < n; ++i) x[i] = x[i] * scale;
}

// kernels/cpu/scale_sum_kernel.cpp:5-22: output += scale[i] * value_i for
// i = 0 .. pos in increasing i, value_i the `size` floats at value + i * stride
// (Armadillo evaluates the product vector, then adds it: two roundings).
void or_scale_sum(const float* value, const float* scale, float* out, int pos, int size, int stride) {
  for (int i = 0; i <= pos; ++i) {
    const float* v = value + (int64_t)i * stride;
    for (int d = 0; d < size; ++d) {
      const float p = scale[i] * v[d];
      out[d] = out[d] + p;
    }
  }
}

// kernels/cpu/swiglu_kernel.cpp:3-23: a = a * (1 / (1 + exp(-a))); out = a * b.
void or_swiglu(const float* a, const float* b, float* out, int n) {
  for (int i = 0; i < n; ++i) {
    const float s = a[i] * (1.0f / (1.0f + std::exp(-a[i])));
    out[i] = s * b[i];
  }
}

// kernels/cpu/add_kernel.cpp:5-19.
void or_add(const float* a, const float* b, float* out, int n) {
  for (int i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

// kernels/cpu/emb_kernel.cpp:4-29: out[i, :] = table[tokens[i], :].  The
// reference rejects only token > vocab (:16), so token == vocab reads past
// the table; the oracle rejects every id outside [0, vocab) and returns -1.
int or_embedding(const int32_t* tokens, int n_tokens, const float* table, int vocab, int dim,
                 float* out) {
  for (int i = 0; i < n_tokens; ++i) {
    const int32_t t = tokens[i];
    if (t < 0 || t >= vocab) return -1;
    std::memcpy(out + (int64_t)i * dim, table + (int64_t)t * dim, sizeof(float) * dim);
  }
  return 0;
}

// sampler/argmax_sampler.cpp:5-13: std::max_element, i.e. the first index of
// the maximum (a later element replaces the best only if strictly greater).
int64_t or_argmax(const float* x, int64_t n) {
  int64_t best = 0;
  for (int64_t i = 1; i < n; ++i) {
    if (x[best] < x[i]) best = i;
  }
  return best;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Model restatement.
// ---------------------------------------------------------------------------
struct or_model {
  int family = 0, quant = 0, group_size = 0;
  int D = 0, Dq = 0, Dkv = 0, F = 0, L = 0, H = 0, KVH = 0, V = 0, S = 0, hd = 0;
  bool tied = false;
  float eps = 1e-5f, theta = 1e4f;
  int rope_style = OR_ROPE_INTERLEAVED;
  const float* emb = nullptr;
  std::vector<const float*> rms_att, rms_ffn, q_norm, k_norm, bq, bk, bv;
  const float* rms_final = nullptr;
  // fp32 matrices or int8 matrices + scales
  std::vector<const void*> wq, wk, wv, wo, w1, w2, w3;
  std::vector<const float*> sq, sk, sv, so, s1, s2, s3;
  const void* wcls = nullptr;
  const float* scls = nullptr;
  std::vector<float> sin_t, cos_t, kcache, vcache;
  std::vector<float> x, xb, q, att, hb, hb2, score, logits;
};

namespace {

void gemv_any(const or_model* m, const void* W, const float* s, const float* x, float* y,
              int rows, int cols) {
  if (m->quant) {
    or_gemv_q8(x, static_cast<const int8_t*>(W), s, y, rows, cols, m->group_size);
  } else {
    or_gemv_f32(x, static_cast<const float*>(W), y, rows, cols, 1.f);
  }
}

}  // namespace

extern "C" {

// Parsing follows model/model.cpp:41-141 (header, derived dims, tied iff
// vocab > 0) and the offset walks of model/llama3.cpp:183-422 (fp32 and int8;
// the int8 Qwen2 walk, model/qwen2.cpp:242-346, is the same and has no bias),
// model/qwen2.cpp:348-485 (bias after each of wq/wk/wv) and
// model/qwen3.cpp:186-299 (8-int header, norms first, q/k norms, lm_head).
or_model* or_model_open(const void* image, size_t size, int family, int quant, char* err,
                        int err_len) {
  auto fail = [&](const char* msg) -> or_model* {
    if (err && err_len > 0) snprintf(err, err_len, "%s", msg);
    return nullptr;
  };
  const bool qwen3 = family == OR_QWEN3;
  const size_t header_ints = qwen3 ? 8 : (quant ? 8 : 7);
  if (size < header_ints * 4) return fail("truncated header");
  const int32_t* h = static_cast<const int32_t*>(image);
  if (qwen3 && quant) return fail("qwen3 has no int8 layout");
  or_model* m = new or_model();
  m->family = family;
  m->quant = quant;
  const int32_t dim = h[0], hidden = h[1];
  m->L = h[2];
  m->H = h[3];
  m->KVH = h[4];
  const int32_t vocab = h[5];
  m->S = h[6];
  if (dim <= 0 || hidden <= 0 || m->L <= 0 || m->H <= 0 || m->KVH <= 0 || vocab == 0 ||
      m->S <= 0 || dim % m->H != 0 || m->H % m->KVH != 0) {
    delete m;
    return fail("bad header values");
  }
  m->V = std::abs(vocab);
  m->hd = dim / m->H;
  m->Dq = dim;
  m->Dkv = dim * m->KVH / m->H;
  if (qwen3) {
    m->D = hidden;
    m->F = h[7];
    m->tied = false;
  } else {
    m->D = dim;
    m->F = hidden;
    m->tied = vocab > 0;
  }
  if (quant) {
    m->group_size = h[7];
    if (m->group_size <= 0) {
      delete m;
      return fail("bad group size");
    }
  }
  switch (family) {
    case OR_LLAMA2: m->eps = 1e-5f; m->theta = 10000.0f; m->rope_style = OR_ROPE_INTERLEAVED; break;
    case OR_LLAMA3: m->eps = 1e-5f; m->theta = 500000.0f; m->rope_style = OR_ROPE_HALF; break;
    case OR_QWEN2: m->eps = 1e-6f; m->theta = 1000000.0f; m->rope_style = OR_ROPE_HALF; break;
    case OR_QWEN3: m->eps = 1e-6f; m->theta = 1000000.0f; m->rope_style = OR_ROPE_HALF; break;
    default: delete m; return fail("unknown family");
  }
  const int L = m->L, D = m->D, Dq = m->Dq, Dkv = m->Dkv, F = m->F, V = m->V, S = m->S;
  const char* base = static_cast<const char*>(image) + header_ints * 4;
  const size_t avail = size - header_ints * 4;
  size_t off = 0;  // bytes from the start of the weight area
  bool overflow = false;
  auto take = [&](size_t bytes) -> const char* {
    const char* p = base + off;
    off += bytes;
    if (off > avail) overflow = true;
    return p;
  };
  auto takef = [&](size_t n) { return reinterpret_cast<const float*>(take(n * 4)); };
  m->rms_att.resize(L);
  m->rms_ffn.resize(L);
  m->wq.resize(L); m->wk.resize(L); m->wv.resize(L); m->wo.resize(L);
  m->w1.resize(L); m->w2.resize(L); m->w3.resize(L);
  if (quant) {
    const int gs = m->group_size;
    m->sq.resize(L); m->sk.resize(L); m->sv.resize(L); m->so.resize(L);
    m->s1.resize(L); m->s2.resize(L); m->s3.resize(L);
    auto takeq = [&](int64_t n, const void** w, const float** s) {
      if (n % gs != 0) overflow = true;
      *w = take(n);
      *s = takef(n / gs);
    };
    for (int l = 0; l < L; ++l) takeq((int64_t)Dq * D, &m->wq[l], &m->sq[l]);
    for (int l = 0; l < L; ++l) takeq((int64_t)Dkv * D, &m->wk[l], &m->sk[l]);
    for (int l = 0; l < L; ++l) takeq((int64_t)Dkv * D, &m->wv[l], &m->sv[l]);
    for (int l = 0; l < L; ++l) takeq((int64_t)D * Dq, &m->wo[l], &m->so[l]);
    for (int l = 0; l < L; ++l) takeq((int64_t)F * D, &m->w1[l], &m->s1[l]);
    for (int l = 0; l < L; ++l) takeq((int64_t)D * F, &m->w2[l], &m->s2[l]);
    for (int l = 0; l < L; ++l) takeq((int64_t)F * D, &m->w3[l], &m->s3[l]);
    if (m->tied) {
      delete m;  // llama3.cpp:258-267 would reinterpret fp32 embedding bytes as int8
      return fail("tied classifier in an int8 image is not supported");
    }
    takeq((int64_t)V * D, &m->wcls, &m->scls);
    m->emb = takef((size_t)V * D);
    for (int l = 0; l < L; ++l) m->rms_att[l] = takef(D);
    for (int l = 0; l < L; ++l) m->rms_ffn[l] = takef(D);
    m->rms_final = takef(D);
  } else if (qwen3) {
    for (int l = 0; l < L; ++l) m->rms_att[l] = takef(D);
    for (int l = 0; l < L; ++l) m->rms_ffn[l] = takef(D);
    m->rms_final = takef(D);
    m->emb = takef((size_t)V * D);
    m->q_norm.resize(L);
    m->k_norm.resize(L);
    for (int l = 0; l < L; ++l) m->wq[l] = takef((size_t)Dq * D);
    for (int l = 0; l < L; ++l) m->q_norm[l] = takef(m->hd);
    for (int l = 0; l < L; ++l) m->wk[l] = takef((size_t)Dkv * D);
    for (int l = 0; l < L; ++l) m->k_norm[l] = takef(m->hd);
    for (int l = 0; l < L; ++l) m->wv[l] = takef((size_t)Dkv * D);
    for (int l = 0; l < L; ++l) m->wo[l] = takef((size_t)D * Dq);
    for (int l = 0; l < L; ++l) m->w1[l] = takef((size_t)F * D);
    for (int l = 0; l < L; ++l) m->w2[l] = takef((size_t)D * F);
    for (int l = 0; l < L; ++l) m->w3[l] = takef((size_t)F * D);
    m->wcls = takef((size_t)V * D);
  } else {
    const bool bias = family == OR_QWEN2;
    m->emb = takef((size_t)V * D);
    for (int l = 0; l < L; ++l) m->rms_att[l] = takef(D);
    if (bias) {
      m->bq.resize(L);
      m->bk.resize(L);
      m->bv.resize(L);
    }
    for (int l = 0; l < L; ++l) {
      m->wq[l] = takef((size_t)Dq * D);
      if (bias) m->bq[l] = takef(Dq);
    }
    for (int l = 0; l < L; ++l) {
      m->wk[l] = takef((size_t)Dkv * D);
      if (bias) m->bk[l] = takef(Dkv);
    }
    for (int l = 0; l < L; ++l) {
      m->wv[l] = takef((size_t)Dkv * D);
      if (bias) m->bv[l] = takef(Dkv);
    }
    for (int l = 0; l < L; ++l) m->wo[l] = takef((size_t)D * Dq);
    for (int l = 0; l < L; ++l) m->rms_ffn[l] = takef(D);
    for (int l = 0; l < L; ++l) m->w1[l] = takef((size_t)F * D);
    for (int l = 0; l < L; ++l) m->w2[l] = takef((size_t)D * F);
    for (int l = 0; l < L; ++l) m->w3[l] = takef((size_t)F * D);
    m->rms_final = takef(D);
    takef((size_t)S * m->hd);  // freq_cos + freq_sin tables, unused by the loaders
    m->wcls = m->tied ? static_cast<const void*>(m->emb) : takef((size_t)V * D);
  }
  if (overflow) {
    delete m;
    return fail("image smaller than the layout its header describes");
  }
  m->sin_t.resize((size_t)S * m->hd);
  m->cos_t.resize((size_t)S * m->hd);
  or_sincos_table(m->hd, S, m->theta, m->sin_t.data(), m->cos_t.data());
  m->kcache.assign((size_t)L * S * Dkv, 0.f);
  m->vcache.assign((size_t)L * S * Dkv, 0.f);
  m->x.resize(D);
  m->xb.resize(std::max(D, Dq));
  m->q.resize(Dq);
  m->att.resize(D);
  m->hb.resize(F);
  m->hb2.resize(F);
  m->score.resize((size_t)m->H * S);
  m->logits.resize(V);
  return m;
}

void or_model_close(or_model* m) { delete m; }

void or_model_dims(const or_model* m, int32_t* o) {
  o[0] = m->D; o[1] = m->Dq; o[2] = m->Dkv; o[3] = m->F; o[4] = m->L;
  o[5] = m->H; o[6] = m->KVH; o[7] = m->V; o[8] = m->S; o[9] = m->hd;
}

// model/llama3.cpp:146-166 (forward), :599-744 (attention_rms, attention_qkv,
// attention_mha, feed_forward, cls_logits); Qwen2 adds the bias add after each
// of wq/wk/wv (op/matmul.cpp:74-77); Qwen3 applies the per-head q and k
// RMSNorm between the projections and RoPE (model/qwen3.cpp:485-500).
int or_model_step(or_model* m, int32_t token, int32_t pos, float* logits) {
  if (pos < 0 || pos >= m->S) return -2;
  if (or_embedding(&token, 1, m->emb, m->V, m->D, m->x.data()) != 0) return -1;
  const int D = m->D, Dq = m->Dq, Dkv = m->Dkv, F = m->F, S = m->S, hd = m->hd;
  float* x = m->x.data();
  float* xb = m->xb.data();
  for (int l = 0; l < m->L; ++l) {
    or_rmsnorm(x, m->rms_att[l], xb, D, m->eps);
    float* kslot = m->kcache.data() + ((size_t)l * S + pos) * Dkv;
    float* vslot = m->vcache.data() + ((size_t)l * S + pos) * Dkv;
    const bool q8 = m->quant != 0;
    gemv_any(m, m->wq[l], q8 ? m->sq[l] : nullptr, xb, m->q.data(), Dq, D);
    if (!m->bq.empty()) or_add(m->q.data(), m->bq[l], m->q.data(), Dq);
    if (m->family == OR_QWEN3) {
      or_rmsnorm_rows(m->q.data(), m->q_norm[l], m->q.data(), Dq / hd, hd, 1e-6f);
    }
    gemv_any(m, m->wk[l], q8 ? m->sk[l] : nullptr, xb, kslot, Dkv, D);
    if (!m->bk.empty()) or_add(kslot, m->bk[l], kslot, Dkv);
    if (m->family == OR_QWEN3) or_rmsnorm_rows(kslot, m->k_norm[l], kslot, Dkv / hd, hd, 1e-6f);
    gemv_any(m, m->wv[l], q8 ? m->sv[l] : nullptr, xb, vslot, Dkv, D);
    if (!m->bv.empty()) or_add(vslot, m->bv[l], vslot, Dkv);
    or_rope(m->rope_style, Dq, Dkv, hd, m->q.data(), kslot, pos, m->sin_t.data(), m->cos_t.data());
    or_mha(pos, m->H, l, S, Dkv, m->H / m->KVH, hd, xb, m->q.data(), m->score.data(),
           m->kcache.data(), m->vcache.data());
    gemv_any(m, m->wo[l], q8 ? m->so[l] : nullptr, xb, m->att.data(), D, Dq);
    or_add(x, m->att.data(), x, D);
    or_rmsnorm(x, m->rms_ffn[l], xb, D, m->eps);
    gemv_any(m, m->w1[l], q8 ? m->s1[l] : nullptr, xb, m->hb.data(), F, D);
    gemv_any(m, m->w3[l], q8 ? m->s3[l] : nullptr, xb, m->hb2.data(), F, D);
    or_swiglu(m->hb.data(), m->hb2.data(), m->hb.data(), F);
    gemv_any(m, m->w2[l], q8 ? m->s2[l] : nullptr, m->hb.data(), m->att.data(), D, F);
    or_add(x, m->att.data(), x, D);
  }
  or_rmsnorm(x, m->rms_final, x, D, m->eps);
  gemv_any(m, m->wcls, m->scls, x, m->logits.data(), m->V, D);
  if (logits) std::memcpy(logits, m->logits.data(), sizeof(float) * m->V);
  return 0;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Batched prompt: the same arithmetic as or_model_step run position after
// position, reorganised so that each weight row is applied to many positions
// while it is in cache.  Every output element is still one dot8 /
// q8_row_dot-ordered sum (8 interleaved accumulators over increasing columns,
// the same fold, the same tail), every per-row operation is the one the step
// calls, and attention of a position reads only the cache rows at or before it,
// which the layer's projections of all earlier positions have written first.
// So the logits and cache rows are bitwise those of the sequential steps
// (pinned by tests/test_oracle.py); only the time differs.
// ---------------------------------------------------------------------------
namespace {

// Y[i][j] = dot8(W_j, X_i) for RB rows of W and TB positions: one ov8
// accumulator per pair holds dot8's 8 interleaved partial sums.
template <int RB, int TB>
void tile_f32(const float* W, int64_t ldw, const float* X, int64_t ldx, int n, float* Y,
              int64_t ldy) {
  ov8 acc[RB][TB];
  for (int j = 0; j < RB; ++j)
    for (int i = 0; i < TB; ++i) acc[j][i] = ov8{0, 0, 0, 0, 0, 0, 0, 0};
  int c = 0;
  for (; c + 8 <= n; c += 8) {
    ov8 w[RB], x[TB];
    for (int j = 0; j < RB; ++j) w[j] = ld8(W + j * ldw + c);
    for (int i = 0; i < TB; ++i) x[i] = ld8(X + i * ldx + c);
    for (int j = 0; j < RB; ++j)
      for (int i = 0; i < TB; ++i) acc[j][i] += w[j] * x[i];
  }
  for (int j = 0; j < RB; ++j)
    for (int i = 0; i < TB; ++i) {
      float s = fold8(acc[j][i]);
      for (int cc = c; cc < n; ++cc) s += W[j * ldw + cc] * X[i * ldx + cc];
      Y[i * ldy + j] = s;
    }
}

template <int RB>
void tile_any(const or_model* m, const void* W, const float* S, int r, int cols, const float* X,
              int64_t ldx, int tb, float* Y, int64_t ldy) {
  if (m->quant) {
    const int gs = m->group_size;
    if (gs % 8 == 0 && cols % 8 == 0) {
      const int8_t* Q = static_cast<const int8_t*>(W);
      switch (tb) {
        case 1: tile_q8<RB, 1>(Q, S, r, cols, gs, X, ldx, Y, ldy); break;
        case 2: tile_q8<RB, 2>(Q, S, r, cols, gs, X, ldx, Y, ldy); break;
        case 3: tile_q8<RB, 3>(Q, S, r, cols, gs, X, ldx, Y, ldy); break;
        default: tile_q8<RB, 4>(Q, S, r, cols, gs, X, ldx, Y, ldy); break;
      }
    } else {
      for (int j = 0; j < RB; ++j)
        for (int i = 0; i < tb; ++i)
          Y[i * ldy + j] = q8_row_dot(X + i * ldx, static_cast<const int8_t*>(W), S,
                                      (int64_t)(r + j) * cols, cols, gs);
    }
    return;
  }
  const float* Wr = static_cast<const float*>(W) + (int64_t)r * cols;
  switch (tb) {
    case 1: tile_f32<RB, 1>(Wr, cols, X, ldx, cols, Y, ldy); break;
    case 2: tile_f32<RB, 2>(Wr, cols, X, ldx, cols, Y, ldy); break;
    case 3: tile_f32<RB, 3>(Wr, cols, X, ldx, cols, Y, ldy); break;
    default: tile_f32<RB, 4>(Wr, cols, X, ldx, cols, Y, ldy); break;
  }
}

// Y[i][r] (row stride ldy) = row r of W applied to X[i] (row stride ldx), for
// i < n and r < rows: the GEMV of gemv_any for each position.  Positions go
// in blocks of 64 (their inputs stay in each core's cache); threads take
// pairs of weight rows, which stay in L1 across a block.
void gemm_rows(const or_model* m, const void* W, const float* S, const float* X, int64_t ldx,
               int n, float* Y, int64_t ldy, int rows, int cols) {
  constexpr int kTB = 64;
  for (int t0 = 0; t0 < n; t0 += kTB) {
    const int tn = std::min(kTB, n - t0);
#pragma omp parallel for schedule(static)
    for (int rp = 0; rp < (rows + 1) / 2; ++rp) {
      const int r = 2 * rp;
      for (int t = t0; t < t0 + tn; t += 4) {
        const int tb = std::min(4, t0 + tn - t);
        const float* Xt = X + (int64_t)t * ldx;
        float* Yt = Y + (int64_t)t * ldy + r;
        if (r + 1 < rows) tile_any<2>(m, W, S, r, cols, Xt, ldx, tb, Yt, ldy);
        else tile_any<1>(m, W, S, r, cols, Xt, ldx, tb, Yt, ldy);
      }
    }
  }
}

}  // namespace

extern "C" {

int or_model_prompt(or_model* m, const int32_t* tokens, int n_tokens, int32_t pos0, float* logits) {
  if (n_tokens <= 0 || pos0 < 0 || (int64_t)pos0 + n_tokens > m->S) return -2;
  for (int i = 0; i < n_tokens; ++i)
    if (tokens[i] < 0 || tokens[i] >= m->V) return -1;
  const int D = m->D, Dq = m->Dq, Dkv = m->Dkv, F = m->F, S = m->S, hd = m->hd, H = m->H;
  const int kv_mul = m->H / m->KVH;
  const bool q8 = m->quant != 0;
  constexpr int kChunk = 512;  // positions per pass (bounds the scratch)
  const int R = std::min(kChunk, n_tokens);
  const int DX = std::max(D, Dq);
  std::vector<float> X((size_t)R * D), XB((size_t)R * DX), Q((size_t)R * Dq), A((size_t)R * D),
      HB((size_t)R * F), HB2((size_t)R * F);
  for (int c0 = 0; c0 < n_tokens; c0 += kChunk) {
    const int n = std::min(kChunk, n_tokens - c0);
    const int p0 = pos0 + c0;
    or_embedding(tokens + c0, n, m->emb, m->V, D, X.data());
    for (int l = 0; l < m->L; ++l) {
      float* kslot = m->kcache.data() + ((size_t)l * S + p0) * Dkv;
      float* vslot = m->vcache.data() + ((size_t)l * S + p0) * Dkv;
#pragma omp parallel for schedule(static)
      for (int i = 0; i < n; ++i)
        or_rmsnorm(&X[(size_t)i * D], m->rms_att[l], &XB[(size_t)i * DX], D, m->eps);
      gemm_rows(m, m->wq[l], q8 ? m->sq[l] : nullptr, XB.data(), DX, n, Q.data(), Dq, Dq, D);
      gemm_rows(m, m->wk[l], q8 ? m->sk[l] : nullptr, XB.data(), DX, n, kslot, Dkv, Dkv, D);
      gemm_rows(m, m->wv[l], q8 ? m->sv[l] : nullptr, XB.data(), DX, n, vslot, Dkv, Dkv, D);
#pragma omp parallel for schedule(static)
      for (int i = 0; i < n; ++i) {
        float* qi = &Q[(size_t)i * Dq];
        float* ki = kslot + (size_t)i * Dkv;
        float* vi = vslot + (size_t)i * Dkv;
        if (!m->bq.empty()) or_add(qi, m->bq[l], qi, Dq);
        if (m->family == OR_QWEN3) or_rmsnorm_rows(qi, m->q_norm[l], qi, Dq / hd, hd, 1e-6f);
        if (!m->bk.empty()) or_add(ki, m->bk[l], ki, Dkv);
        if (m->family == OR_QWEN3) or_rmsnorm_rows(ki, m->k_norm[l], ki, Dkv / hd, hd, 1e-6f);
        if (!m->bv.empty()) or_add(vi, m->bv[l], vi, Dkv);
        or_rope(m->rope_style, Dq, Dkv, hd, qi, ki, p0 + i, m->sin_t.data(), m->cos_t.data());
      }
      const float* kl = m->kcache.data() + (size_t)l * S * Dkv;
      const float* vl = m->vcache.data() + (size_t)l * S * Dkv;
#pragma omp parallel
      {
        std::vector<float> sc(S);
#pragma omp for schedule(dynamic, 1)
        for (int ih = 0; ih < n * H; ++ih) {
          const int i = n - 1 - ih / H, h = ih % H;  // the longest rows first
          mha_head(p0 + i, h, Dkv, kv_mul, hd, &XB[(size_t)i * DX + (size_t)h * hd],
                   &Q[(size_t)i * Dq + (size_t)h * hd], sc.data(), kl, vl);
        }
      }
      gemm_rows(m, m->wo[l], q8 ? m->so[l] : nullptr, XB.data(), DX, n, A.data(), D, D, Dq);
#pragma omp parallel for schedule(static)
      for (int i = 0; i < n; ++i) {
        float* xi = &X[(size_t)i * D];
        or_add(xi, &A[(size_t)i * D], xi, D);
        or_rmsnorm(xi, m->rms_ffn[l], &XB[(size_t)i * DX], D, m->eps);
      }
      gemm_rows(m, m->w1[l], q8 ? m->s1[l] : nullptr, XB.data(), DX, n, HB.data(), F, F, D);
      gemm_rows(m, m->w3[l], q8 ? m->s3[l] : nullptr, XB.data(), DX, n, HB2.data(), F, F, D);
#pragma omp parallel for schedule(static)
      for (int i = 0; i < n; ++i)
        or_swiglu(&HB[(size_t)i * F], &HB2[(size_t)i * F], &HB[(size_t)i * F], F);
      gemm_rows(m, m->w2[l], q8 ? m->s2[l] : nullptr, HB.data(), F, n, A.data(), D, D, F);
#pragma omp parallel for schedule(static)
      for (int i = 0; i < n; ++i) or_add(&X[(size_t)i * D], &A[(size_t)i * D], &X[(size_t)i * D], D);
    }
    if (c0 + n == n_tokens) {
      float* x = m->x.data();
      std::memcpy(x, &X[(size_t)(n - 1) * D], sizeof(float) * D);
      or_rmsnorm(x, m->rms_final, x, D, m->eps);
      gemv_any(m, m->wcls, m->scls, x, m->logits.data(), m->V, D);
    }
  }
  if (logits) std::memcpy(logits, m->logits.data(), sizeof(float) * m->V);
  return 0;
}

// demo/main.cpp:5-47: prompt positions 0..P-2 run without sampling; from
// position P-1 on, the current token is embedded, the step runs and the
// argmax becomes the next token.  `next` starts at prompt[0]
// (demo/main_qwen3.cpp:93), which keeps a 1-token prompt well defined.
int or_model_generate(or_model* m, const int32_t* prompt, int P, int n_new, int32_t* out_tokens) {
  if (P <= 0 || n_new <= 0) return 0;
  // Positions 0..P-1 all take prompt tokens (at P-1 through the decode
  // branch, whose `next` is prompt[P-1]); they run as one batched prompt,
  // bitwise equal to stepping them one by one.
  if (or_model_prompt(m, prompt, P, 0, nullptr) != 0) return -1;
  int32_t next = static_cast<int32_t>(or_argmax(m->logits.data(), m->V));
  int n_out = 0;
  out_tokens[n_out++] = next;
  for (int pos = P; pos < P + n_new - 1; ++pos) {
    if (or_model_step(m, next, pos, nullptr) != 0) return -1;
    next = static_cast<int32_t>(or_argmax(m->logits.data(), m->V));
    out_tokens[n_out++] = next;
  }
  return n_out;
}

void or_model_kv_row(const or_model* m, int layer, int pos, int which_v, float* out) {
  const std::vector<float>& c = which_v ? m->vcache : m->kcache;
  std::memcpy(out, c.data() + ((size_t)layer * m->S + pos) * m->Dkv, sizeof(float) * m->Dkv);
}

}  // extern "C"
