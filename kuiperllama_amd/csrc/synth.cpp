// Synthetic model images in the reference's .bin byte layouts.
//
// Layouts (offsets in the order the writers emit them):
//  * fp32 Llama v0  -- tools/export_llama.py:79-131: header 7 x int32
//    {dim, hidden, layers, heads, kv_heads, +-vocab, seq_len} (negative vocab
//    = separate classifier), embedding, attention norms, wq, wk, wv, wo, ffn
//    norms, w1, w2, w3, final norm, freq_cos + freq_sin [seq_len x hd/2 each],
//    classifier if not tied.
//  * int8 Llama     -- tools/export_llama.py:134-210: header 8 x int32 (+group
//    size), every matrix as int8[n] followed by fp32 scales[n / group], in the
//    order wq, wk, wv, wo, w1, w2, w3, classifier, then fp32 embedding,
//    attention norms, ffn norms, final norm.
//  * fp32 Qwen2     -- tools/export_qwen2.py:79-134: the v0 layout with each
//    of wq / wk / wv followed by its bias.
//  * fp32 Qwen3     -- tools/export_qwen3.py:55-102: header 8 x int32
//    {q_dim, dim, layers, heads, kv_heads, vocab, seq_len, ffn}, norms
//    (attention [L], ffn [L], final), embedding, wq, q_norm, wk, k_norm, wv,
//    wo, w1 (gate), w2 (down), w3 (up), lm_head.
//  * int8 Qwen2     -- tools/export_qwen2.py:137-210: the int8 Llama layout
//    (no biases: the int8 loader model/qwen2.cpp:242-346 reads none).
//
// Values: N(0, stddev) for matrices, embeddings and biases; norm weights
// (attention, ffn, final, Qwen3 q/k) 1.0, or 1 + N(0, norm_stddev) when the
// spec asks for it, one stream per norm role and layer; zeros for the freq
// tables (the loaders skip them).  The normal stream of a tensor depends only
// on (seed, role, layer, element index), so a model's fp32 and int8 images
// hold the same underlying weights.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include <algorithm>
#include <thread>

#include "kuiper_hip.h"

namespace {

int default_threads() {
  const unsigned n = std::thread::hardware_concurrency();
  return n == 0 ? 1 : static_cast<int>(std::min(n, 64u));
}

// Static block partition of [0, n) over n_threads std::threads.
template <typename Fn>
void parallel_for(int64_t n, int n_threads, Fn fn) {
  if (n_threads <= 1 || n < 4096) {
    for (int64_t i = 0; i < n; ++i) fn(i);
    return;
  }
  const int64_t per = (n + n_threads - 1) / n_threads;
  std::vector<std::thread> pool;
  for (int t = 0; t < n_threads; ++t) {
    const int64_t b = t * per, e = std::min(n, b + per);
    if (b >= e) break;
    pool.emplace_back([=] {
      for (int64_t i = b; i < e; ++i) fn(i);
    });
  }
  for (auto& th : pool) th.join();
}

enum Role : int32_t {
  kEmb = 1, kWq = 2, kWk = 3, kWv = 4, kWo = 5, kW1 = 6, kW2 = 7, kW3 = 8, kCls = 9,
  kBq = 10, kBk = 11, kBv = 12,
  kRmsAtt = 13, kRmsFfn = 14, kRmsFinal = 15, kQNorm = 16, kKNorm = 17
};

inline uint64_t mix64(uint64_t z) {
  // splitmix64 finaliser (Steele, Lea, Flood: "Fast splittable pseudorandom
  // number generators", 2014).
  z += 0x9e3779b97f4a7c15ULL;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

// Box-Muller on two 24-bit uniforms in float (tails reach 5.8 sigma, ample for
// N(0, 0.02) weights); one 64-bit hash per uniform.
void normal_stream(uint64_t seed, int32_t role, int32_t layer, float stddev, float* out,
                   int64_t n, int n_threads) {
  const uint64_t key = mix64(seed ^ mix64((uint64_t(uint32_t(role)) << 32) | uint32_t(layer)));
  const int64_t pairs = (n + 1) / 2;
  const float two_pi = 6.28318530717958647692f;
  const float inv24 = 1.0f / 16777216.0f;
  parallel_for(pairs, n_threads, [&](int64_t j) {
    const uint64_t a = mix64(key + 2 * uint64_t(j));
    const uint64_t b = mix64(key + 2 * uint64_t(j) + 1);
    const float u1 = static_cast<float>((a >> 40) + 1) * inv24;  // (0, 1]
    const float u2 = static_cast<float>(b >> 40) * inv24;        // [0, 1)
    const float r = std::sqrt(-2.0f * std::log(u1)) * stddev;
    const float t = two_pi * u2;
    out[2 * j] = r * std::cos(t);
    if (2 * j + 1 < n) out[2 * j + 1] = r * std::sin(t);
  });
}

// tools/export_llama.py:49-73 (quantize_q80): per contiguous group, scale =
// max|w| / 127 in fp32, q = round-half-even(w / scale).  A group of zeros
// (scale 0) quantises to q = 0.
void quantize_groups(const float* w, int64_t n, int gs, int8_t* q, float* scales, int n_threads) {
  const int64_t groups = n / gs;
  parallel_for(groups, n_threads, [&](int64_t g) {
    const float* wg = w + g * gs;
    float wmax = 0.f;
    for (int i = 0; i < gs; ++i) wmax = std::fmax(wmax, std::fabs(wg[i]));
    const float scale = wmax / 127.0f;
    scales[g] = scale;
    for (int i = 0; i < gs; ++i) {
      const float v = scale == 0.f ? 0.f : std::nearbyint(wg[i] / scale);
      q[g * gs + i] = static_cast<int8_t>(v);
    }
  });
}

struct Dims {
  int64_t D, Dq, Dkv, F, L, H, KVH, V, S, hd, gs;
  bool tied, qwen3, qwen2, q8;
  float norm_std;
};

int derive(const kl_model_spec* s, Dims* d) {
  if (!s) return KL_EINVAL;
  if (s->family < KL_FAMILY_LLAMA2 || s->family > KL_FAMILY_QWEN3) return KL_EINVAL;
  if (s->dim <= 0 || s->q_dim <= 0 || s->hidden_dim <= 0 || s->layers <= 0 || s->heads <= 0 ||
      s->kv_heads <= 0 || s->vocab <= 0 || s->seq_len <= 0)
    return KL_EINVAL;
  if (s->q_dim % s->heads != 0 || s->heads % s->kv_heads != 0) return KL_EINVAL;
  d->qwen3 = s->family == KL_FAMILY_QWEN3;
  d->qwen2 = s->family == KL_FAMILY_QWEN2;
  d->q8 = s->group_size > 0;
  if (!d->qwen3 && s->q_dim != s->dim) return KL_EINVAL;
  if (d->q8 && (d->qwen3 || s->tied)) return KL_EUNSUPP;
  if (!(s->norm_stddev >= 0.f)) return KL_EINVAL;
  d->norm_std = s->norm_stddev;
  d->D = s->dim;
  d->Dq = s->q_dim;
  d->H = s->heads;
  d->KVH = s->kv_heads;
  d->hd = d->Dq / d->H;
  d->Dkv = d->Dq * d->KVH / d->H;
  d->F = s->hidden_dim;
  d->L = s->layers;
  d->V = s->vocab;
  d->S = s->seq_len;
  d->gs = s->group_size;
  d->tied = s->tied != 0 && !d->qwen3;
  if (d->q8) {
    const int64_t mats[] = {d->Dq * d->D, d->Dkv * d->D, d->F * d->D, d->V * d->D};
    for (int64_t n : mats)
      if (n % d->gs != 0) return KL_EINVAL;
  }
  return KL_OK;
}

int64_t image_size(const Dims& d) {
  const int64_t L = d.L;
  if (d.qwen3) {
    int64_t f = (2 * L + 1) * d.D + d.V * d.D;
    f += L * (d.Dq * d.D + d.hd + d.Dkv * d.D + d.hd + d.Dkv * d.D + d.D * d.Dq);
    f += L * 3 * d.F * d.D + d.V * d.D;
    return 8 * 4 + f * 4;
  }
  if (d.q8) {
    auto qbytes = [&](int64_t n) { return n + (n / d.gs) * 4; };
    int64_t b = 8 * 4;
    b += L * (qbytes(d.Dq * d.D) + 2 * qbytes(d.Dkv * d.D) + qbytes(d.D * d.Dq));
    b += L * 3 * qbytes(d.F * d.D);
    b += qbytes(d.V * d.D);  // untied classifier
    b += (d.V * d.D + (2 * L + 1) * d.D) * 4;
    return b;
  }
  int64_t f = d.V * d.D + L * d.D;
  f += L * (d.Dq * d.D + 2 * d.Dkv * d.D + d.D * d.Dq);
  if (d.qwen2) f += L * (d.Dq + 2 * d.Dkv);
  f += L * d.D + L * 3 * d.F * d.D + d.D + d.S * d.hd;
  if (!d.tied) f += d.V * d.D;
  return 7 * 4 + f * 4;
}

class Writer {
 public:
  Writer(char* base, int64_t cap, uint64_t seed, float stddev, int threads)
      : base_(base), cap_(cap), seed_(seed), stddev_(stddev), threads_(threads) {}
  bool ok() const { return ok_; }
  int64_t offset() const { return off_; }
  void header(const int32_t* h, int n) { put(h, 4 * n); }
  void normal(int32_t role, int32_t layer, int64_t n) {
    float* p = reinterpret_cast<float*>(reserve(n * 4));
    if (p) normal_stream(seed_, role, layer, stddev_, p, n, threads_);
  }
  // A norm weight vector: 1.0, or 1 + N(0, norm_std) from the (role, layer)
  // stream.
  void norm(int32_t role, int32_t layer, int64_t n, float norm_std) {
    float* p = reinterpret_cast<float*>(reserve(n * 4));
    if (!p) return;
    if (norm_std == 0.f) {
      for (int64_t i = 0; i < n; ++i) p[i] = 1.f;
      return;
    }
    normal_stream(seed_, role, layer, norm_std, p, n, threads_);
    for (int64_t i = 0; i < n; ++i) p[i] += 1.f;
  }
  void fill(float v, int64_t n) {
    float* p = reinterpret_cast<float*>(reserve(n * 4));
    if (!p) return;
    for (int64_t i = 0; i < n; ++i) p[i] = v;
  }
  void quantized(int32_t role, int32_t layer, int64_t n, int gs) {
    scratch_.resize(n);
    normal_stream(seed_, role, layer, stddev_, scratch_.data(), n, threads_);
    int8_t* q = reinterpret_cast<int8_t*>(reserve(n));
    float* s = reinterpret_cast<float*>(reserve((n / gs) * 4));
    if (q && s) quantize_groups(scratch_.data(), n, gs, q, s, threads_);
  }

 private:
  void put(const void* src, int64_t bytes) {
    char* p = reserve(bytes);
    if (p) std::memcpy(p, src, bytes);
  }
  char* reserve(int64_t bytes) {
    if (!ok_ || off_ + bytes > cap_) {
      ok_ = false;
      return nullptr;
    }
    char* p = base_ + off_;
    off_ += bytes;
    return p;
  }
  char* base_;
  int64_t cap_;
  int64_t off_ = 0;
  uint64_t seed_;
  float stddev_;
  int threads_;
  bool ok_ = true;
  std::vector<float> scratch_;
};

}  // namespace

extern "C" {

int kl_synth_image_size(const kl_model_spec* spec, int64_t* bytes) {
  Dims d;
  const int rc = derive(spec, &d);
  if (rc != KL_OK) return rc;
  if (!bytes) return KL_EINVAL;
  *bytes = image_size(d);
  return KL_OK;
}

int kl_synth_normal(uint64_t seed, int32_t role, int32_t layer, float stddev, float* out,
                    int64_t n) {
  if (!out || n < 0) return KL_EINVAL;
  normal_stream(seed, role, layer, stddev, out, n, default_threads());
  return KL_OK;
}

int kl_quantize_q8(const float* w, int64_t n, int group_size, int8_t* q, float* scales) {
  if (!w || !q || !scales || group_size <= 0 || n % group_size != 0) return KL_EINVAL;
  quantize_groups(w, n, group_size, q, scales, default_threads());
  return KL_OK;
}

int kl_synth_image(const kl_model_spec* spec, uint64_t seed, float stddev, void* out,
                   int64_t out_bytes, int n_threads) {
  Dims d;
  int rc = derive(spec, &d);
  if (rc != KL_OK) return rc;
  if (!out || out_bytes < image_size(d)) return KL_EINVAL;
  if (n_threads <= 0) n_threads = default_threads();
  Writer w(static_cast<char*>(out), out_bytes, seed, stddev, n_threads);
  const int32_t L = static_cast<int32_t>(d.L);
  if (d.qwen3) {
    const int32_t h[8] = {int32_t(d.Dq), int32_t(d.D), L, int32_t(d.H), int32_t(d.KVH),
                          int32_t(d.V), int32_t(d.S), int32_t(d.F)};
    w.header(h, 8);
    for (int32_t l = 0; l < L; ++l) w.norm(kRmsAtt, l, d.D, d.norm_std);
    for (int32_t l = 0; l < L; ++l) w.norm(kRmsFfn, l, d.D, d.norm_std);
    w.norm(kRmsFinal, 0, d.D, d.norm_std);
    w.normal(kEmb, 0, d.V * d.D);
    for (int32_t l = 0; l < L; ++l) w.normal(kWq, l, d.Dq * d.D);
    for (int32_t l = 0; l < L; ++l) w.norm(kQNorm, l, d.hd, d.norm_std);
    for (int32_t l = 0; l < L; ++l) w.normal(kWk, l, d.Dkv * d.D);
    for (int32_t l = 0; l < L; ++l) w.norm(kKNorm, l, d.hd, d.norm_std);
    for (int32_t l = 0; l < L; ++l) w.normal(kWv, l, d.Dkv * d.D);
    for (int32_t l = 0; l < L; ++l) w.normal(kWo, l, d.D * d.Dq);
    for (int32_t l = 0; l < L; ++l) w.normal(kW1, l, d.F * d.D);
    for (int32_t l = 0; l < L; ++l) w.normal(kW2, l, d.D * d.F);
    for (int32_t l = 0; l < L; ++l) w.normal(kW3, l, d.F * d.D);
    w.normal(kCls, 0, d.V * d.D);
  } else if (d.q8) {
    const int32_t h[8] = {int32_t(d.D), int32_t(d.F), L, int32_t(d.H), int32_t(d.KVH),
                          -int32_t(d.V), int32_t(d.S), int32_t(d.gs)};
    w.header(h, 8);
    const int gs = static_cast<int>(d.gs);
    for (int32_t l = 0; l < L; ++l) w.quantized(kWq, l, d.Dq * d.D, gs);
    for (int32_t l = 0; l < L; ++l) w.quantized(kWk, l, d.Dkv * d.D, gs);
    for (int32_t l = 0; l < L; ++l) w.quantized(kWv, l, d.Dkv * d.D, gs);
    for (int32_t l = 0; l < L; ++l) w.quantized(kWo, l, d.D * d.Dq, gs);
    for (int32_t l = 0; l < L; ++l) w.quantized(kW1, l, d.F * d.D, gs);
    for (int32_t l = 0; l < L; ++l) w.quantized(kW2, l, d.D * d.F, gs);
    for (int32_t l = 0; l < L; ++l) w.quantized(kW3, l, d.F * d.D, gs);
    w.quantized(kCls, 0, d.V * d.D, gs);
    w.normal(kEmb, 0, d.V * d.D);
    for (int32_t l = 0; l < L; ++l) w.norm(kRmsAtt, l, d.D, d.norm_std);
    for (int32_t l = 0; l < L; ++l) w.norm(kRmsFfn, l, d.D, d.norm_std);
    w.norm(kRmsFinal, 0, d.D, d.norm_std);
  } else {
    const int32_t vocab = d.tied ? int32_t(d.V) : -int32_t(d.V);
    const int32_t h[7] = {int32_t(d.D), int32_t(d.F), L, int32_t(d.H), int32_t(d.KVH), vocab,
                          int32_t(d.S)};
    w.header(h, 7);
    w.normal(kEmb, 0, d.V * d.D);
    for (int32_t l = 0; l < L; ++l) w.norm(kRmsAtt, l, d.D, d.norm_std);
    for (int32_t l = 0; l < L; ++l) {
      w.normal(kWq, l, d.Dq * d.D);
      if (d.qwen2) w.normal(kBq, l, d.Dq);
    }
    for (int32_t l = 0; l < L; ++l) {
      w.normal(kWk, l, d.Dkv * d.D);
      if (d.qwen2) w.normal(kBk, l, d.Dkv);
    }
    for (int32_t l = 0; l < L; ++l) {
      w.normal(kWv, l, d.Dkv * d.D);
      if (d.qwen2) w.normal(kBv, l, d.Dkv);
    }
    for (int32_t l = 0; l < L; ++l) w.normal(kWo, l, d.D * d.Dq);
    for (int32_t l = 0; l < L; ++l) w.norm(kRmsFfn, l, d.D, d.norm_std);
    for (int32_t l = 0; l < L; ++l) w.normal(kW1, l, d.F * d.D);
    for (int32_t l = 0; l < L; ++l) w.normal(kW2, l, d.D * d.F);
    for (int32_t l = 0; l < L; ++l) w.normal(kW3, l, d.F * d.D);
    w.norm(kRmsFinal, 0, d.D, d.norm_std);
    w.fill(0.f, d.S * d.hd);
    if (!d.tied) w.normal(kCls, 0, d.V * d.D);
  }
  if (!w.ok() || w.offset() != image_size(d)) return KL_EFORMAT;
  return KL_OK;
}

}  // extern "C"
