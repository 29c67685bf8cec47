// Model, the layer-by-layer decode step on the HIP kernels, and the fused
// path on the persistent decode engine (the reference's source/model/
// {model,llama3,qwen2,qwen3}.cpp and demo/main.cpp, for kDeviceHIP).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>

#include "kuiper/model.h"
#include "kuiper_hip.h"

namespace model {

RawModelData::~RawModelData() {
  if (data != nullptr && data != MAP_FAILED) munmap(data, file_size);
  if (fd != -1) close(fd);
}

void DecoderLayers::to_hip(const std::shared_ptr<kernel::HipConfig>& config) {
  auto move = [&](const std::shared_ptr<op::Layer>& layer) {
    if (!layer) return;
    layer->set_hip_config(config);
    layer->to_hip();
  };
  move(add_layer_);
  move(rope_layer_);
  move(swiglu_layer_);
  move(mha_layer_);
  move(cls_layer_);
  move(embedding_layer_);
  for (auto* group : {&wq_layers_, &wk_layers_, &wv_layers_, &wo_layers_, &w1_layers_,
                      &w2_layers_, &w3_layers_, &rmsnorm_layers_})
    for (auto& layer : *group) move(layer);
}

namespace {
kernel::KernelTraits traits_of(ModelFamily family) {
  kernel::KernelTraits t;
  switch (family) {
    case ModelFamily::kLlama2: t.rope_style = KL_ROPE_INTERLEAVED; t.rope_theta = 1e4f; t.rms_eps = 1e-5f; break;
    case ModelFamily::kLlama3: t.rope_style = KL_ROPE_HALF; t.rope_theta = 5e5f; t.rms_eps = 1e-5f; break;
    case ModelFamily::kQwen2:
    case ModelFamily::kQwen3: t.rope_style = KL_ROPE_HALF; t.rope_theta = 1e6f; t.rms_eps = 1e-6f; break;
  }
  t.rms_dim_eps = 1e-6f;
  return t;
}
}  // namespace

Model::Model(base::TokenizerType tokenizer_type, base::ModelType model_type,
             std::string token_path, std::string model_path, bool is_quant_model,
             ModelFamily family)
    : is_quant_model_(is_quant_model),
      family_(family),
      token_path_(std::move(token_path)),
      model_path_(std::move(model_path)),
      model_type_(model_type),
      tokenizer_type_(tokenizer_type) {}

LLama2Model::LLama2Model(base::TokenizerType tokenizer_type, std::string token_path,
                         std::string model_path, bool is_quant_model, ModelFamily family)
    : Model(tokenizer_type, base::ModelType::kModelTypeLLama2, std::move(token_path),
            std::move(model_path), is_quant_model, family) {}

Qwen2Model::Qwen2Model(base::TokenizerType tokenizer_type, std::string token_path,
                       std::string model_path, bool is_quant_model)
    : LLama2Model(tokenizer_type, std::move(token_path), std::move(model_path), is_quant_model,
                  ModelFamily::kQwen2) {}

Qwen3Model::Qwen3Model(base::TokenizerType tokenizer_type, std::string token_path,
                       std::string model_path, bool is_quant_model)
    : LLama2Model(tokenizer_type, std::move(token_path), std::move(model_path), is_quant_model,
                  ModelFamily::kQwen3) {}

Model::~Model() {
  if (engine_) kl_engine_destroy(engine_);
  engine_ = nullptr;
  for (void* ev : profile_all_events_) kl_event_destroy(ev);
  // Layers and buffers release their device memory before the stream goes.
  layers_.reset();
  buffers_.clear();
  sampler_.reset();
}

template <class Fn>
void Model::profiled(const char* name, Fn&& fn, void* stream) const {
  if (!profiling_) {
    fn();
    return;
  }
  auto take = [&]() {
    void* ev = nullptr;
    if (!profile_events_.empty()) {
      ev = profile_events_.back();
      profile_events_.pop_back();
    } else {
      KUIPER_CHECK(kl_event_create(&ev) == KL_OK, "kl_event_create failed");
      profile_all_events_.push_back(ev);
    }
    return ev;
  };
  void* start = take();
  void* stop = take();
  void* st = stream ? stream : hip_config_->stream;
  KUIPER_CHECK(kl_event_record(start, st) == KL_OK, "kl_event_record failed");
  fn();
  KUIPER_CHECK(kl_event_record(stop, st) == KL_OK, "kl_event_record failed");
  profile_pending_.push_back({name, start, stop});
}

// Waits for the streams and adds the pending operations' device times.
void Model::resolve_profile() const {
  if (profile_pending_.empty()) return;
  KUIPER_CHECK(kl_device_sync() == KL_OK, "kl_device_sync failed");
  for (const ProfileRecord& r : profile_pending_) {
    float ms = 0.f;
    KUIPER_CHECK(kl_event_elapsed_ms(r.start, r.stop, &ms) == KL_OK, "kl_event_elapsed_ms failed");
    auto& acc = profile_[r.name];
    acc.first += ms;
    acc.second += 1;
    profile_events_.push_back(r.start);
    profile_events_.push_back(r.stop);
  }
  profile_pending_.clear();
}

void Model::reset_profile_stats() const {
  resolve_profile();
  profile_.clear();
  profiling_ = true;
}

std::vector<OpProfileStat> Model::get_profile_stats() const {
  resolve_profile();
  std::vector<OpProfileStat> out;
  for (const auto& [name, acc] : profile_) {
    OpProfileStat st;
    st.op_name = name;
    st.total_ms = acc.first;
    st.calls = acc.second;
    st.avg_ms = acc.second ? acc.first / static_cast<double>(acc.second) : 0.0;
    out.push_back(st);
  }
  return out;
}

// llama3.cpp:111-145 for kDeviceHIP.  The tokenizer is optional (token ids in
// and out), so an empty token_path is accepted; a given one must load.
base::Status LLama2Model::init(base::DeviceType device_type) {
  if (device_type != base::DeviceType::kDeviceHIP)
    return base::error::InvalidArgument(
        "This backend runs on kDeviceHIP only; the CPU and CUDA paths are the reference's.");
  device_type_ = device_type;
  // The file is parsed and sized before any device work, so a bad path or
  // image is reported without touching the GPU.
  base::Status s = read_model_file();
  if (!s) return s;
  if (!token_path_.empty()) {
    s = create_encode_layer();
    if (!s) return s;
  }
  s = create_layers();
  if (!s) return s;
  if (kl_set_device(0) != KL_OK) return base::error::InternalError("kl_set_device(0) failed.");
  hip_config_ = std::make_shared<kernel::HipConfig>();
  if (hip_config_->create() != KL_OK)
    return base::error::InternalError("The HIP stream could not be created.");
  kernel::set_kernel_traits(traits_of(family_));
  init_mem();
  kernel::sin_cos_cache_calc_hip(config_->head_size_, config_->seq_len_,
                                 get_buffer(ModelBufferType::kSinCache),
                                 get_buffer(ModelBufferType::kCosCache));
  sampler_ = std::make_unique<sampler::ArgmaxSampler>(device_type_);
  return base::error::Success();
}

// Qwen3 images are fp32 only (qwen3.cpp has no int8 loader).
base::Status Qwen3Model::init(base::DeviceType device_type) {
  if (is_quant_model_) return base::error::InvalidArgument("Qwen3 images have no int8 layout.");
  return LLama2Model::init(device_type);
}

// model.cpp:41-111: header, optional group size, then mmap of the whole file.
// Qwen3 images carry an eighth header int (the FFN width).
base::Status Model::read_model_file() {
  if (model_path_.empty())
    return base::error::PathNotValid("No model file was given (empty path).");
  auto raw = std::make_shared<RawModelData>();
  raw->fd = open(model_path_.c_str(), O_RDONLY);
  if (raw->fd == -1)
    return base::error::PathNotValid("Cannot open model file " + model_path_ + ".");
  struct stat st;
  if (fstat(raw->fd, &st) == -1)
    return base::error::ModelParseError("Cannot stat model file " + model_path_ + ".");
  raw->file_size = static_cast<size_t>(st.st_size);
  const bool qwen3 = family_ == ModelFamily::kQwen3;
  const size_t header_ints = 7 + ((qwen3 || is_quant_model_) ? 1 : 0);
  if (raw->file_size < header_ints * sizeof(int32_t))
    return base::error::ModelParseError(
        "Model file too short for its header.");
  raw->data = mmap(nullptr, raw->file_size, PROT_READ, MAP_PRIVATE, raw->fd, 0);
  if (raw->data == MAP_FAILED || raw->data == nullptr) {
    raw->data = nullptr;
    return base::error::ModelParseError("Cannot mmap model file " + model_path_ + ".");
  }
  const int32_t* h = static_cast<const int32_t*>(raw->data);
  ModelConfig config;
  config.dim = h[0];
  config.hidden_dim = h[1];
  config.layer_num = h[2];
  config.head_num = h[3];
  config.kv_head_num = h[4];
  config.vocab_size = h[5];
  config.seq_len = h[6];
  int32_t extra = 0;
  if (is_quant_model_) group_size_ = h[7];
  if (qwen3) extra = h[7];
  base::Status s = generate_model_infos(config, extra);
  if (!s) return s;
  if (is_quant_model_ && group_size_ <= 0)
    return base::error::ModelParseError(
        "Model file too short for the int8 group size field.");
  raw->weight_data = static_cast<const int8_t*>(raw->data) + header_ints * sizeof(int32_t);
  raw_model_data_ = raw;
  return base::error::Success();
}

// model.cpp:113-141 (Qwen3: qwen3.cpp's header {q_dim, dim, ..., ffn}).
base::Status Model::generate_model_infos(const ModelConfig& c, int32_t extra) {
  if (c.dim <= 0 || c.hidden_dim <= 0 || c.layer_num <= 0 || c.head_num <= 0 ||
      c.kv_head_num <= 0 || c.vocab_size == 0 || c.seq_len <= 0 || c.dim % c.head_num != 0 ||
      c.head_num % c.kv_head_num != 0)
    return base::error::ModelParseError("The model header is not valid.");
  auto cfg = std::make_unique<TransformerConfig>();
  cfg->layer_num_ = c.layer_num;
  cfg->head_num_ = c.head_num;
  cfg->kv_head_num_ = c.kv_head_num;
  cfg->seq_len_ = c.seq_len;
  cfg->head_size_ = c.dim / c.head_num;
  cfg->kv_dim_ = c.dim * c.kv_head_num / c.head_num;
  cfg->kv_mul_ = c.head_num / c.kv_head_num;
  cfg->q_dim_ = c.dim;
  cfg->dim_ = c.dim;
  cfg->hidden_dim_ = c.hidden_dim;
  cfg->is_shared_weight_ = c.vocab_size > 0;
  cfg->vocab_size_ = std::abs(c.vocab_size);
  config_ = std::move(cfg);
  return base::error::Success();
}

// qwen3.cpp's header {q_dim, dim, layers, heads, kv_heads, vocab, seq_len,
// ffn_dim}: the first int sizes the heads, the second is the model width,
// the eighth the FFN width; the classifier is always a separate lm_head.
base::Status Qwen3Model::generate_model_infos(const ModelConfig& c, int32_t extra) {
  if (extra <= 0) return base::error::ModelParseError("The Qwen3 FFN width is not valid.");
  base::Status s = Model::generate_model_infos(c, extra);
  if (!s) return s;
  config_->dim_ = c.hidden_dim;
  config_->hidden_dim_ = extra;
  config_->is_shared_weight_ = false;
  return base::error::Success();
}

namespace {
// Wraps consecutive tensors of the weight region as external CPU weights of
// new layers, advancing through the file.
struct WeightWalk {
  const float* p;
  base::DeviceType dev;
  std::shared_ptr<op::Layer> matmul(int32_t rows, int32_t cols, bool bias = false) {
    const auto cpu = base::DeviceType::kDeviceCPU;
    auto m = std::make_shared<op::MatmulLayer>(dev, rows, cols, false, bias);
    m->set_weight(0, {rows, cols}, p, cpu);
    p += static_cast<size_t>(rows) * cols;
    if (bias) {
      int32_t n = rows;
      m->set_bias(0, n, p, cpu);
      p += rows;
    }
    return m;
  }
  std::shared_ptr<op::Layer> norm(int32_t n) {
    auto r = std::make_shared<op::RmsNormLayer>(dev, n);
    r->set_weight(0, {n}, p, base::DeviceType::kDeviceCPU);
    p += n;
    return r;
  }
  std::shared_ptr<op::Layer> embedding(int32_t V, int32_t D, int32_t seq_len) {
    auto e = std::make_shared<op::EmbeddingLayer>(dev, D, seq_len, V);
    e->set_weight(0, {V, D}, p, base::DeviceType::kDeviceCPU);
    p += static_cast<size_t>(V) * D;
    return e;
  }
};
}  // namespace

void LLama2Model::create_param_layers() { create_param_layers_fp32(false); }

void Qwen2Model::create_param_layers() { create_param_layers_fp32(true); }

// Walks the fp32 weight region in file order (llama3.cpp:289-422; with
// biases, qwen2.cpp:348-485), wrapping each tensor as an external CPU weight.
void LLama2Model::create_param_layers_fp32(bool bias) {
  const auto& c = *config_;
  const int32_t L = c.layer_num_, D = c.dim_, Dq = c.q_dim_, Dkv = c.kv_dim_, F = c.hidden_dim_,
                V = c.vocab_size_, hd = c.head_size_;
  WeightWalk w{reinterpret_cast<const float*>(raw_model_data_->weight_data), device_type_};
  auto& ly = *layers_;
  ly.embedding_layer_ = w.embedding(V, D, c.seq_len_);
  std::vector<std::shared_ptr<op::Layer>> att, ffn;
  for (int32_t l = 0; l < L; ++l) att.push_back(w.norm(D));
  for (int32_t l = 0; l < L; ++l) ly.wq_layers_.push_back(w.matmul(Dq, D, bias));
  for (int32_t l = 0; l < L; ++l) ly.wk_layers_.push_back(w.matmul(Dkv, D, bias));
  for (int32_t l = 0; l < L; ++l) ly.wv_layers_.push_back(w.matmul(Dkv, D, bias));
  for (int32_t l = 0; l < L; ++l) ly.wo_layers_.push_back(w.matmul(D, Dq));
  for (int32_t l = 0; l < L; ++l) ffn.push_back(w.norm(D));
  for (int32_t l = 0; l < L; ++l) ly.w1_layers_.push_back(w.matmul(F, D));
  for (int32_t l = 0; l < L; ++l) ly.w2_layers_.push_back(w.matmul(D, F));
  for (int32_t l = 0; l < L; ++l) ly.w3_layers_.push_back(w.matmul(F, D));
  auto final_norm = w.norm(D);
  w.p += static_cast<size_t>(c.seq_len_) * hd;  // freq_cis_real + freq_cis_imag, unused
  if (c.is_shared_weight_) {
    auto cls = std::make_shared<op::MatmulLayer>(device_type_, V, D);
    cls->set_weight(0, {V, D},
                    std::static_pointer_cast<op::LayerParam>(ly.embedding_layer_)
                        ->get_weight(0)
                        .ptr<float>(),
                    base::DeviceType::kDeviceCPU);
    ly.cls_layer_ = cls;
  } else {
    ly.cls_layer_ = w.matmul(V, D);
  }
  for (auto& x : att) ly.rmsnorm_layers_.push_back(x);
  for (auto& x : ffn) ly.rmsnorm_layers_.push_back(x);
  ly.rmsnorm_layers_.push_back(final_norm);
}

// qwen3.cpp:186-299: the norms first, the embedding, then per kind of matrix
// all layers (q norms after wq, k norms after wk) and the lm_head; the q/k
// norms go to rmsnorm slots 2L+1 .. 4L.
void Qwen3Model::create_param_layers() {
  const auto& c = *config_;
  const int32_t L = c.layer_num_, D = c.dim_, Dq = c.q_dim_, Dkv = c.kv_dim_, F = c.hidden_dim_,
                V = c.vocab_size_, hd = c.head_size_;
  WeightWalk w{reinterpret_cast<const float*>(raw_model_data_->weight_data), device_type_};
  auto& ly = *layers_;
  for (int32_t i = 0; i < 2 * L + 1; ++i) ly.rmsnorm_layers_.push_back(w.norm(D));
  ly.embedding_layer_ = w.embedding(V, D, c.seq_len_);
  std::vector<std::shared_ptr<op::Layer>> qn, kn;
  for (int32_t l = 0; l < L; ++l) ly.wq_layers_.push_back(w.matmul(Dq, D));
  for (int32_t l = 0; l < L; ++l) qn.push_back(w.norm(hd));
  for (int32_t l = 0; l < L; ++l) ly.wk_layers_.push_back(w.matmul(Dkv, D));
  for (int32_t l = 0; l < L; ++l) kn.push_back(w.norm(hd));
  for (int32_t l = 0; l < L; ++l) ly.wv_layers_.push_back(w.matmul(Dkv, D));
  for (int32_t l = 0; l < L; ++l) ly.wo_layers_.push_back(w.matmul(D, Dq));
  for (int32_t l = 0; l < L; ++l) ly.w1_layers_.push_back(w.matmul(F, D));
  for (int32_t l = 0; l < L; ++l) ly.w2_layers_.push_back(w.matmul(D, F));
  for (int32_t l = 0; l < L; ++l) ly.w3_layers_.push_back(w.matmul(F, D));
  ly.cls_layer_ = w.matmul(V, D);
  for (auto& x : qn) ly.rmsnorm_layers_.push_back(x);
  for (auto& x : kn) ly.rmsnorm_layers_.push_back(x);
}

// llama3.cpp:183-287 (and qwen2.cpp:242-346, the same walk without biases):
// int8 matrices, each followed by its fp32 group scales, then the fp32
// embedding and norm weights.
void LLama2Model::create_param_quant_layers() {
  const auto& c = *config_;
  const int32_t L = c.layer_num_, D = c.dim_, Dq = c.q_dim_, Dkv = c.kv_dim_, F = c.hidden_dim_,
                V = c.vocab_size_;
  const auto cpu = base::DeviceType::kDeviceCPU;
  const auto dev = device_type_;
  const int8_t* p = raw_model_data_->weight_data;
  auto& ly = *layers_;
  auto qmatmul = [&](int32_t rows, int32_t cols) {
    auto m = std::make_shared<op::MatmulLayer>(dev, rows, cols, true);
    m->set_group_size(group_size_);
    m->set_weight(0, {rows, cols}, p, cpu);
    p += static_cast<size_t>(rows) * cols + m->get_scale_num() * sizeof(float);
    return m;
  };
  for (int32_t l = 0; l < L; ++l) ly.wq_layers_.push_back(qmatmul(Dq, D));
  for (int32_t l = 0; l < L; ++l) ly.wk_layers_.push_back(qmatmul(Dkv, D));
  for (int32_t l = 0; l < L; ++l) ly.wv_layers_.push_back(qmatmul(Dkv, D));
  for (int32_t l = 0; l < L; ++l) ly.wo_layers_.push_back(qmatmul(D, Dq));
  for (int32_t l = 0; l < L; ++l) ly.w1_layers_.push_back(qmatmul(F, D));
  for (int32_t l = 0; l < L; ++l) ly.w2_layers_.push_back(qmatmul(D, F));
  for (int32_t l = 0; l < L; ++l) ly.w3_layers_.push_back(qmatmul(F, D));
  ly.cls_layer_ = qmatmul(V, D);
  const float* f = reinterpret_cast<const float*>(p);
  auto emb = std::make_shared<op::EmbeddingLayer>(dev, D, c.seq_len_, V);
  emb->set_weight(0, {V, D}, f, cpu);
  f += static_cast<size_t>(V) * D;
  ly.embedding_layer_ = emb;
  for (int32_t i = 0; i < 2 * L + 1; ++i) {
    auto r = std::make_shared<op::RmsNormLayer>(dev, D);
    r->set_weight(0, {D}, f, cpu);
    f += D;
    ly.rmsnorm_layers_.push_back(r);
  }
}

void LLama2Model::create_nonparam_layers() {
  const auto& c = *config_;
  auto& ly = *layers_;
  ly.rope_layer_ = std::make_shared<op::RoPELayer>(device_type_, c.q_dim_, c.kv_dim_, c.head_size_);
  ly.mha_layer_ = std::make_shared<op::MultiHeadAttention>(
      device_type_, 0, c.kv_mul_, c.kv_dim_, c.seq_len_, c.head_num_, c.head_size_);
  ly.add_layer_ = std::make_shared<op::VecAddLayer>(device_type_);
  ly.swiglu_layer_ = std::make_shared<op::SwiGLULayer>(device_type_, c.hidden_dim_);
}

// Bytes of the fp32 layouts after the header (export_llama.py:79-210 with
// biases for Qwen2, export_qwen3.py:55-102).
size_t LLama2Model::fp32_weight_bytes() const {
  const auto& c = *config_;
  const size_t L = c.layer_num_, D = c.dim_, Dq = c.q_dim_, Dkv = c.kv_dim_, F = c.hidden_dim_,
               V = c.vocab_size_, hd = c.head_size_;
  return 4 * (V * D + L * (2 * D + Dq * D + 2 * Dkv * D + D * Dq + 3 * F * D) + D +
              static_cast<size_t>(c.seq_len_) * hd + (c.is_shared_weight_ ? 0 : V * D));
}

size_t Qwen2Model::fp32_weight_bytes() const {
  const auto& c = *config_;
  return LLama2Model::fp32_weight_bytes() +
         4 * static_cast<size_t>(c.layer_num_) * (c.q_dim_ + 2 * static_cast<size_t>(c.kv_dim_));
}

size_t Qwen3Model::fp32_weight_bytes() const {
  const auto& c = *config_;
  const size_t L = c.layer_num_, D = c.dim_, Dq = c.q_dim_, Dkv = c.kv_dim_, F = c.hidden_dim_,
               V = c.vocab_size_, hd = c.head_size_;
  return 4 * ((2 * L + 1) * D + V * D + L * (Dq * D + 2 * hd + 2 * Dkv * D + D * Dq + 3 * F * D) +
              V * D);
}

// llama3.cpp:499-575: sizes the image, creates every layer and checks them.
base::Status LLama2Model::create_layers() {
  const auto& c = *config_;
  const size_t L = c.layer_num_, D = c.dim_, Dq = c.q_dim_, Dkv = c.kv_dim_, F = c.hidden_dim_,
               V = c.vocab_size_;
  size_t need = 0;  // bytes after the header
  if (is_quant_model_) {
    if (c.is_shared_weight_)
      return base::error::ModelParseError(
          "A tied classifier is not defined for int8 images (the classifier is int8).");
    const size_t gs = group_size_;
    auto q8 = [&](size_t n) { return n + (n / gs) * 4; };
    for (size_t n : {Dq * D, Dkv * D, Dkv * D, D * Dq, F * D, D * F, F * D})
      if (n % gs) return base::error::ModelParseError("A matrix is not a multiple of the group size.");
    need = L * (q8(Dq * D) + 2 * q8(Dkv * D) + q8(D * Dq) + 2 * q8(F * D) + q8(D * F)) +
           q8(V * D) + 4 * (V * D + (2 * L + 1) * D);
  } else {
    need = fp32_weight_bytes();
  }
  const size_t have = raw_model_data_->file_size -
                      (raw_model_data_->weight_data - static_cast<const int8_t*>(raw_model_data_->data));
  if (need > have)
    return base::error::ModelParseError("The weight file is shorter than its header implies.");

  layers_ = std::make_unique<DecoderLayers>();
  if (is_quant_model_) create_param_quant_layers();
  else create_param_layers();
  create_nonparam_layers();

  auto& ly = *layers_;
  if (!ly.embedding_layer_)
    return base::error::InternalError("The model has no embedding layer after loading.");
  const size_t norms = family_ == ModelFamily::kQwen3 ? 4 * L + 1 : 2 * L + 1;
  if (ly.rmsnorm_layers_.size() != norms)
    return base::error::InternalError("The model has the wrong number of norm layers after loading.");
  if (ly.wq_layers_.size() != L || ly.wk_layers_.size() != L || ly.wv_layers_.size() != L ||
      ly.wo_layers_.size() != L)
    return base::error::InternalError("An attention projection is missing after loading.");
  if (ly.w1_layers_.size() != L || ly.w2_layers_.size() != L || ly.w3_layers_.size() != L)
    return base::error::InternalError("A feed-forward projection is missing after loading.");
  if (!ly.cls_layer_ || !ly.rope_layer_ || !ly.mha_layer_ || !ly.add_layer_ || !ly.swiglu_layer_)
    return base::error::InternalError("The model layers are incomplete after loading.");
  return base::error::Success();
}

base::Status Model::insert_buffer(ModelBufferType buffer_idx, const tensor::Tensor& tensor) {
  if (buffers_.count(buffer_idx) > 0)
    return base::error::KeyHasExits("model buffer " + std::to_string(int(buffer_idx)) +
                                    " is registered already");
  if (tensor.is_empty())
    return base::error::InvalidArgument("An empty tensor cannot be registered as a model buffer.");
  buffers_.insert({buffer_idx, tensor});
  return base::error::Success();
}

tensor::Tensor& Model::get_buffer(ModelBufferType buffer_idx) {
  KUIPER_CHECK(buffers_.count(buffer_idx) > 0, "buffer " + std::to_string(int(buffer_idx)));
  return buffers_.at(buffer_idx);
}

const tensor::Tensor& Model::get_buffer(ModelBufferType buffer_idx) const {
  KUIPER_CHECK(buffers_.count(buffer_idx) > 0, "buffer " + std::to_string(int(buffer_idx)));
  return buffers_.at(buffer_idx);
}

// llama3.cpp:424-497 (Qwen3: qwen3.cpp:301-380): moves the layers to the
// device and lays out the step's buffers with the reference's aliases.  The
// score buffer is the reference's [head_num x seq_len] floats, uninitialised
// (llama3.cpp:485-487); the attention kernel keeps its split partials in it.
void LLama2Model::init_mem() {
  const auto& c = *config_;
  auto alloc = base::HIPDeviceAllocatorFactory::get_instance();
  auto alloc_cpu = base::CPUDeviceAllocatorFactory::get_instance();
  layers_->to_hip(hip_config_);
  void* stream = hip_config_->stream;
  using T = tensor::Tensor;
  using DT = base::DataType;

  T input_tokens(DT::kDataTypeInt32, 1, true, alloc_cpu);
  T input_embeddings(DT::kDataTypeFp32, 1, c.dim_, true, alloc);
  T sin_cache(DT::kDataTypeFp32, c.head_size_ * c.seq_len_, true, alloc);
  T cos_cache(DT::kDataTypeFp32, c.head_size_ * c.seq_len_, true, alloc);
  STATUS_CHECK(insert_buffer(ModelBufferType::kSinCache, sin_cache));
  STATUS_CHECK(insert_buffer(ModelBufferType::kCosCache, cos_cache));
  STATUS_CHECK(insert_buffer(ModelBufferType::kInputTokens, input_tokens));
  STATUS_CHECK(insert_buffer(ModelBufferType::kInputEmbeddings, input_embeddings));

  // The reference's aliases (llama3.cpp:455-459, :486-488) where the widths
  // agree; separate buffers where the heads' width differs from the model's
  // (Qwen3, qwen3.cpp:301-380).
  const bool separate = c.q_dim_ != c.dim_;
  T rms_output(DT::kDataTypeFp32, c.dim_, true, alloc);
  STATUS_CHECK(insert_buffer(ModelBufferType::kOutputRMSNorm, rms_output));
  if (separate) {
    T out_mha(DT::kDataTypeFp32, c.q_dim_, true, alloc);
    STATUS_CHECK(insert_buffer(ModelBufferType::kOutputMHA, out_mha));
  } else {
    STATUS_CHECK(insert_buffer(ModelBufferType::kOutputMHA, rms_output));
  }
  STATUS_CHECK(insert_buffer(ModelBufferType::kW2Output, rms_output));
  STATUS_CHECK(insert_buffer(ModelBufferType::kFFNRMSNorm, rms_output));

  T w1_output(DT::kDataTypeFp32, c.hidden_dim_, true, alloc);
  T w3_output(DT::kDataTypeFp32, c.hidden_dim_, true, alloc);
  STATUS_CHECK(insert_buffer(ModelBufferType::kW1Output, w1_output));
  STATUS_CHECK(insert_buffer(ModelBufferType::kW3Output, w3_output));

  T key_cache(DT::kDataTypeFp32, c.layer_num_, c.seq_len_, c.kv_dim_, true, alloc);
  T value_cache(DT::kDataTypeFp32, c.layer_num_, c.seq_len_, c.kv_dim_, true, alloc);
  KUIPER_CHECK(!key_cache.is_empty() && !value_cache.is_empty(), "KV cache allocation");
  alloc->memset_zero(key_cache.ptr<void>(), key_cache.byte_size(), stream);
  alloc->memset_zero(value_cache.ptr<void>(), value_cache.byte_size(), stream);
  STATUS_CHECK(insert_buffer(ModelBufferType::kKeyCache, key_cache));
  STATUS_CHECK(insert_buffer(ModelBufferType::kValueCache, value_cache));

  T query(DT::kDataTypeFp32, c.q_dim_, true, alloc);
  STATUS_CHECK(insert_buffer(ModelBufferType::kQuery, query));

  T pos_tensor(DT::kDataTypeInt32, 1, true, alloc_cpu);
  STATUS_CHECK(insert_buffer(ModelBufferType::kInputPos, pos_tensor));

  const size_t ws = kernel::mha_workspace_bytes(c.head_num_, c.kv_mul_, c.seq_len_, c.head_size_);
  T attn(DT::kDataTypeFp32, c.head_num_, c.seq_len_, true, alloc);
  KUIPER_CHECK(attn.byte_size() >= ws, "attention partials exceed the score buffer");
  STATUS_CHECK(insert_buffer(ModelBufferType::kScoreStorage, attn));
  if (separate) {
    T attn_output(DT::kDataTypeFp32, c.dim_, true, alloc);
    STATUS_CHECK(insert_buffer(ModelBufferType::kAttnOutput, attn_output));
  } else {
    STATUS_CHECK(insert_buffer(ModelBufferType::kAttnOutput, query));
  }

  T forward_output(DT::kDataTypeFp32, c.vocab_size_, true, alloc);
  T forward_output_cpu(DT::kDataTypeFp32, c.vocab_size_, true, alloc_cpu);
  STATUS_CHECK(insert_buffer(ModelBufferType::kForwardOutputCPU, forward_output_cpu));
  STATUS_CHECK(insert_buffer(ModelBufferType::kForwardOutput, forward_output));
  KUIPER_CHECK(kl_stream_sync(stream) == KL_OK, "init_mem sync");
}

std::pair<tensor::Tensor, tensor::Tensor> Model::slice_kv_cache(int32_t layer_idx,
                                                                int32_t token_pos) const {
  const auto& c = *config_;
  KUIPER_CHECK(layer_idx >= 0 && layer_idx < c.layer_num_ && token_pos >= 0 &&
                   token_pos < c.seq_len_,
               "KV slot out of range");
  const int64_t offset = (static_cast<int64_t>(layer_idx) * c.seq_len_ + token_pos) * c.kv_dim_;
  float* k = const_cast<float*>(get_buffer(ModelBufferType::kKeyCache).ptr<float>(offset));
  float* v = const_cast<float*>(get_buffer(ModelBufferType::kValueCache).ptr<float>(offset));
  tensor::Tensor key(base::DataType::kDataTypeFp32, c.kv_dim_, false, nullptr, k);
  tensor::Tensor val(base::DataType::kDataTypeFp32, c.kv_dim_, false, nullptr, v);
  key.set_device_type(device_type_);
  val.set_device_type(device_type_);
  return {key, val};
}

// llama3.cpp:577-597
op::EmbeddingOutput LLama2Model::embedding(const std::vector<int>& tokens) const {
  KUIPER_CHECK(!tokens.empty(), "no tokens to embed");
  auto* self = const_cast<LLama2Model*>(this);
  tensor::Tensor& input_tokens = self->get_buffer(ModelBufferType::kInputTokens);
  tensor::Tensor& input_embeddings = self->get_buffer(ModelBufferType::kInputEmbeddings);
  const int32_t n = static_cast<int32_t>(tokens.size());
  if (input_tokens.size() != tokens.size()) {
    input_tokens.reshape({n});
    input_embeddings.reshape({n, config_->dim_});
  }
  for (int32_t i = 0; i < n; ++i) input_tokens.index<int32_t>(i) = tokens[i];
  tensor::Tensor input_token_num(base::DataType::kDataTypeInt32, n);
  profiled("input.embedding", [&] {
    STATUS_CHECK(layers_->embedding_layer_->forward(input_tokens, input_token_num, input_embeddings));
  });
  resolve_profile();
  return op::EmbeddingOutput(input_tokens, input_embeddings, input_token_num);
}

// model.cpp:240-265
tensor::Tensor Model::fill_input(const tensor::Tensor& pos_tensor,
                                 const op::EmbeddingOutput& embedding_output,
                                 bool is_prompt) const {
  const int32_t pos = pos_tensor.index<int32_t>(0);
  const int32_t index = is_prompt ? pos : 0;
  const auto& emb = embedding_output.input_embeddings;
  KUIPER_CHECK(index >= 0 && static_cast<size_t>(index + 1) * config_->dim_ <= emb.size(),
               "fill_input row out of range");
  auto buffer = std::make_shared<base::Buffer>(
      config_->dim_ * sizeof(float), nullptr,
      const_cast<float*>(emb.ptr<float>(static_cast<int64_t>(index) * config_->dim_)), true);
  tensor::Tensor input(base::DataType::kDataTypeFp32, config_->dim_);
  input.assign(buffer);
  input.set_device_type(device_type_);
  return input;
}

// The layer-by-layer step (llama3.cpp:146-166, :599-744; qwen2/qwen3 alike),
// with the reference's profile names (qwen2.cpp:648-800).
void LLama2Model::attention_rms(int32_t layer_idx, const tensor::Tensor& input) const {
  profiled("attn.rmsnorm", [&] {
    STATUS_CHECK(layers_->rmsnorm_layers_.at(layer_idx)->forward(
        input, get_buffer(ModelBufferType::kOutputRMSNorm)));
  });
}

void LLama2Model::attention_qkv(int32_t layer_idx, const tensor::Tensor& pos_tensor) const {
  tensor::Tensor query = get_buffer(ModelBufferType::kQuery);
  const int32_t pos = pos_tensor.index<int32_t>(0);
  auto [key, val] = slice_kv_cache(layer_idx, pos);
  const tensor::Tensor& rms = get_buffer(ModelBufferType::kOutputRMSNorm);
  profiled("attn.wq", [&] { STATUS_CHECK(layers_->wq_layers_.at(layer_idx)->forward(rms, query)); });
  profiled("attn.wk", [&] { STATUS_CHECK(layers_->wk_layers_.at(layer_idx)->forward(rms, key)); });
  profiled("attn.wv", [&] { STATUS_CHECK(layers_->wv_layers_.at(layer_idx)->forward(rms, val)); });
  profiled("attn.rope", [&] {
    STATUS_CHECK(layers_->rope_layer_->forward(query, key, pos_tensor,
                                               get_buffer(ModelBufferType::kSinCache),
                                               get_buffer(ModelBufferType::kCosCache),
                                               tensor::Tensor{}));
  });
}

// qwen3.cpp:459-513: the per-head q/k RMSNorm (rows of head_size, norm
// layers 2L+1+l and 3L+1+l) between the projections and RoPE.
void Qwen3Model::attention_qkv(int32_t layer_idx, const tensor::Tensor& pos_tensor) const {
  const auto& c = *config_;
  tensor::Tensor query = get_buffer(ModelBufferType::kQuery);
  const int32_t pos = pos_tensor.index<int32_t>(0);
  auto [key, val] = slice_kv_cache(layer_idx, pos);
  const tensor::Tensor& rms = get_buffer(ModelBufferType::kOutputRMSNorm);
  profiled("attn.wq", [&] { STATUS_CHECK(layers_->wq_layers_.at(layer_idx)->forward(rms, query)); });
  query.reshape({c.q_dim_ / c.head_size_, c.head_size_});
  profiled("attn.q_norm", [&] {
    STATUS_CHECK(layers_->rmsnorm_layers_.at(layer_idx + 2 * c.layer_num_ + 1)->forward(query, query));
  });
  query.reshape({c.q_dim_});
  profiled("attn.wk", [&] { STATUS_CHECK(layers_->wk_layers_.at(layer_idx)->forward(rms, key)); });
  key.reshape({c.kv_dim_ / c.head_size_, c.head_size_});
  profiled("attn.k_norm", [&] {
    STATUS_CHECK(layers_->rmsnorm_layers_.at(layer_idx + 3 * c.layer_num_ + 1)->forward(key, key));
  });
  key.reshape({c.kv_dim_});
  profiled("attn.wv", [&] { STATUS_CHECK(layers_->wv_layers_.at(layer_idx)->forward(rms, val)); });
  profiled("attn.rope", [&] {
    STATUS_CHECK(layers_->rope_layer_->forward(query, key, pos_tensor,
                                               get_buffer(ModelBufferType::kSinCache),
                                               get_buffer(ModelBufferType::kCosCache),
                                               tensor::Tensor{}));
  });
}

void LLama2Model::attention_mha(int32_t layer_idx, const tensor::Tensor& pos_tensor) const {
  const tensor::Tensor& mha_output = get_buffer(ModelBufferType::kOutputMHA);
  auto mha = std::static_pointer_cast<op::MultiHeadAttention>(layers_->mha_layer_);
  mha->set_pos(pos_tensor.index<int32_t>(0));
  mha->set_layer_idx(layer_idx);
  profiled("attn.mha", [&] {
    STATUS_CHECK(mha->forward(get_buffer(ModelBufferType::kQuery),
                              get_buffer(ModelBufferType::kScoreStorage),
                              get_buffer(ModelBufferType::kKeyCache),
                              get_buffer(ModelBufferType::kValueCache), mha_output));
  });
  profiled("attn.wo", [&] {
    STATUS_CHECK(layers_->wo_layers_.at(layer_idx)->forward(
        mha_output, get_buffer(ModelBufferType::kAttnOutput)));
  });
}

void LLama2Model::feed_forward(int32_t layer_idx, const tensor::Tensor& input) const {
  const auto& c = *config_;
  profiled("ffn.residual_add1", [&] {
    STATUS_CHECK(layers_->add_layer_->forward(input, get_buffer(ModelBufferType::kAttnOutput), input));
  });
  const tensor::Tensor& ffn_norm = get_buffer(ModelBufferType::kFFNRMSNorm);
  profiled("ffn.rmsnorm", [&] {
    STATUS_CHECK(layers_->rmsnorm_layers_.at(layer_idx + c.layer_num_)->forward(input, ffn_norm));
  });
  const tensor::Tensor& w1 = get_buffer(ModelBufferType::kW1Output);
  const tensor::Tensor& w3 = get_buffer(ModelBufferType::kW3Output);
  profiled("ffn.w1", [&] { STATUS_CHECK(layers_->w1_layers_.at(layer_idx)->forward(ffn_norm, w1)); });
  profiled("ffn.w3", [&] { STATUS_CHECK(layers_->w3_layers_.at(layer_idx)->forward(ffn_norm, w3)); });
  profiled("ffn.swiglu", [&] { STATUS_CHECK(layers_->swiglu_layer_->forward(w1, w3, w1)); });
  const tensor::Tensor& w2 = get_buffer(ModelBufferType::kW2Output);
  profiled("ffn.w2", [&] { STATUS_CHECK(layers_->w2_layers_.at(layer_idx)->forward(w1, w2)); });
  profiled("ffn.residual_add2", [&] { STATUS_CHECK(layers_->add_layer_->forward(input, w2, input)); });
}

void LLama2Model::cls_logits(const tensor::Tensor& input) const {
  profiled("output.rmsnorm", [&] {
    STATUS_CHECK(layers_->rmsnorm_layers_.at(2 * config_->layer_num_)->forward(input, input));
  });
  profiled("output.cls", [&] {
    STATUS_CHECK(layers_->cls_layer_->forward(input, get_buffer(ModelBufferType::kForwardOutput)));
  });
}

int32_t LLama2Model::post_processing(const tensor::Tensor&, bool is_prompt) const {
  const tensor::Tensor& out = get_buffer(ModelBufferType::kForwardOutput);
  if (is_prompt) return -1;
  int32_t next = -1;
  profiled("sampler.argmax", [&] {
    next = static_cast<int32_t>(sampler_->sample(out.ptr<float>(), out.size(), hip_config_->stream));
  });
  return next;
}

base::Status LLama2Model::forward(const tensor::Tensor& input, const tensor::Tensor& pos_tensor,
                            int&) const {
  if (input.is_empty()) return base::error::InvalidArgument("The input tensor is empty.");
  const int32_t pos = pos_tensor.index<int32_t>(0);
  if (pos < 0 || pos >= config_->seq_len_)
    return base::error::InvalidArgument("The position is outside the sequence length.");
  for (int32_t l = 0; l < config_->layer_num_; ++l) {
    attention_rms(l, input);
    attention_qkv(l, pos_tensor);
    attention_mha(l, pos_tensor);
    feed_forward(l, input);
  }
  cls_logits(input);
  return base::error::Success();
}

// llama3.cpp:641-649.  Fused: the token is the one embedding() stored for
// this input row (fill_input's row of kInputEmbeddings), and the engine runs
// the whole step in one launch; its logits are copied into kForwardOutput.
base::Status LLama2Model::predict(const tensor::Tensor& input, const tensor::Tensor& pos_tensor,
                            bool is_prompt, int& next) const {
  if (!fused_) {
    base::Status s = forward(input, pos_tensor, next);
    if (!s) return s;
    next = post_processing(pos_tensor, is_prompt);
    resolve_profile();
    return base::error::Success();
  }
  const int32_t pos = pos_tensor.index<int32_t>(0);
  if (pos < 0 || pos >= config_->seq_len_)
    return base::error::InvalidArgument("The position is outside the sequence length.");
  const int32_t row = is_prompt ? pos : 0;
  const tensor::Tensor& tokens = get_buffer(ModelBufferType::kInputTokens);
  const tensor::Tensor& emb = get_buffer(ModelBufferType::kInputEmbeddings);
  if (row >= static_cast<int32_t>(tokens.size()) ||
      input.ptr<float>() != emb.ptr<float>(static_cast<int64_t>(row) * config_->dim_))
    return base::error::InvalidArgument(
        "The fused step takes the input row that fill_input() returned for embedding().");
  int32_t sampled = -1;
  int rc = KL_OK;
  void* est = nullptr;
  kl_engine_stream(engine_, &est);
  profiled("fused.step", [&] { rc = kl_engine_step(engine_, tokens.index<int32_t>(row), pos, &sampled, nullptr); },
           est);
  if (rc != KL_OK) return base::error::InternalError(std::string("kl_engine_step: ") + kl_error_string(rc));
  const float* d_logits = nullptr;
  kl_engine_buffers(engine_, &d_logits, nullptr, nullptr);
  const tensor::Tensor& out = get_buffer(ModelBufferType::kForwardOutput);
  rc = kl_memcpy_d2d(const_cast<float*>(out.ptr<float>()), d_logits, out.byte_size(),
                     hip_config_->stream);
  if (rc == KL_OK) rc = kl_stream_sync(hip_config_->stream);
  if (rc != KL_OK) return base::error::InternalError("logits copy failed");
  resolve_profile();
  next = is_prompt ? -1 : sampled;
  return base::error::Success();
}

// Creates the engine from the mapped image on first use.  Switching modes
// starts a new sequence: each path keeps its own KV cache.
base::Status Model::set_fused(bool enable) {
  if (!raw_model_data_) return base::error::InvalidArgument("init() has not run.");
  if (enable && !engine_) {
    int rc = kl_engine_create(raw_model_data_->data, raw_model_data_->file_size,
                              static_cast<int>(family_), is_quant_model_ ? 1 : 0, &engine_);
    if (rc != KL_OK) {
      engine_ = nullptr;
      return base::error::InternalError(std::string("kl_engine_create: ") + kl_error_string(rc));
    }
  }
  fused_ = enable;
  return base::error::Success();
}

// demo/main.cpp:5-47 without the tokenizer: positions 0..P-2 are prompt steps,
// position P-1 feeds the last prompt token through the decode branch, and
// n_new tokens are sampled (no end-of-sequence stop: there is no tokenizer).
// Fused: the whole loop runs on the device (kl_engine_generate).
base::Status Model::generate(const std::vector<int32_t>& prompt, int32_t n_new,
                             std::vector<int32_t>& out) const {
  const int32_t P = static_cast<int32_t>(prompt.size());
  if (P < 1 || n_new < 1 || P + n_new - 1 > config_->seq_len_)
    return base::error::InvalidArgument("prompt + new tokens must fit the sequence length.");
  out.assign(n_new, -1);
  if (fused_) {
    int rc = kl_engine_generate(engine_, prompt.data(), P, n_new, out.data(), nullptr);
    if (rc != KL_OK) return base::error::InternalError(std::string("kl_engine_generate: ") + kl_error_string(rc));
    return base::error::Success();
  }
  const op::EmbeddingOutput prompt_embedding = embedding(prompt);
  tensor::Tensor pos_tensor = get_buffer(ModelBufferType::kInputPos);
  int next = -1;
  for (int32_t pos = 0; pos < P - 1; ++pos) {
    pos_tensor.index<int32_t>(0) = pos;
    base::Status s = predict(fill_input(pos_tensor, prompt_embedding, true), pos_tensor, true, next);
    if (!s) return s;
  }
  int32_t token = prompt[P - 1];
  for (int32_t i = 0; i < n_new; ++i) {
    const int32_t pos = P - 1 + i;
    pos_tensor.index<int32_t>(0) = pos;
    const op::EmbeddingOutput emb = embedding({token});
    base::Status s = predict(fill_input(pos_tensor, emb, false), pos_tensor, false, next);
    if (!s) return s;
    out[i] = next;
    token = next;
  }
  return base::error::Success();
}

base::Status Model::set_prefill(bool enable) {
  if (enable && !fused_) return base::error::InvalidArgument("prefill needs set_fused(true)");
  const int rc = kl_engine_set_prefill(engine_, enable ? 1 : 0);
  if (rc != KL_OK)
    return base::error::FunctionNotImplement(std::string("kl_engine_set_prefill: ") +
                                             kl_error_string(rc));
  prefill_ = enable;
  return base::error::Success();
}

base::Status Model::prefill(const std::vector<int32_t>& prompt, int& next) const {
  if (!fused_ || !engine_) return base::error::InvalidArgument("prefill needs set_fused(true)");
  if (prompt.empty() || static_cast<int32_t>(prompt.size()) > config_->seq_len_)
    return base::error::InvalidArgument("The prompt does not fit the sequence length.");
  int32_t nx = -1;
  float ms = 0.f;
  int rc = kl_engine_prefill(engine_, prompt.data(), static_cast<int>(prompt.size()), &nx, nullptr,
                             &ms);
  if (rc != KL_OK)
    return base::error::InternalError(std::string("kl_engine_prefill: ") + kl_error_string(rc));
  if (profiling_) {  // the engine times the batched pass on its stream
    auto& acc = profile_["prefill.batched"];
    acc.first += ms;
    acc.second += 1;
  }
  const float* d_logits = nullptr;
  kl_engine_buffers(engine_, &d_logits, nullptr, nullptr);
  const tensor::Tensor& out = get_buffer(ModelBufferType::kForwardOutput);
  rc = kl_memcpy_d2d(const_cast<float*>(out.ptr<float>()), d_logits, out.byte_size(),
                     hip_config_->stream);
  if (rc == KL_OK) rc = kl_stream_sync(hip_config_->stream);
  if (rc != KL_OK) return base::error::InternalError("logits copy failed");
  next = nx;
  return base::error::Success();
}

// model.cpp:143-173, the layer chosen by tokenizer type and model family
// rather than build flags.  Unlike the reference, the vocabulary size stays
// the image's (Qwen tokenizers hold fewer ids than the embedding has rows);
// a tokenizer with more ids than the model is refused.
base::Status Model::create_encode_layer() {
  if (tokenizer_type_ == base::TokenizerType::kEncodeSpe) {
    encode_layer_ = std::make_unique<op::SpeEncodeLayer>(token_path_, true, false);
  } else if (tokenizer_type_ == base::TokenizerType::kEncodeBpe) {
    if (family_ == ModelFamily::kQwen2 || family_ == ModelFamily::kQwen3)
      encode_layer_ = std::make_unique<op::QwenEncodeLayer>(token_path_, false, false);
    else
      encode_layer_ = std::make_unique<op::BpeEncodeLayer>(token_path_, true, false);
  } else {
    return base::error::InvalidArgument("A tokenizer file was given without a tokenizer type.");
  }
  base::Status s = encode_layer_->init();
  if (!s) {
    encode_layer_.reset();
    return s;
  }
  if (encode_layer_->vocab_size() <= 0 || encode_layer_->vocab_size() > config_->vocab_size_) {
    encode_layer_.reset();
    return base::error::ModelParseError("The tokenizer's vocabulary does not fit the model's.");
  }
  return base::error::Success();
}

bool Model::is_sentence_ending(int32_t token_idx) const {
  if (encode_layer_ && encode_layer_->is_sentence_ending(token_idx)) return true;
  for (int32_t e : eos_tokens_)
    if (e == token_idx) return true;
  return false;
}
std::string Model::decode(int32_t token_idx) const {
  return encode_layer_ ? encode_layer_->decode(token_idx) : std::string();
}
std::string Model::decode(std::vector<int32_t> token_idxs) const {
  return encode_layer_ ? encode_layer_->decode(token_idxs) : std::string();
}
std::vector<int32_t> Model::encode(const std::string& sentence) const {
  if (encode_layer_) return encode_layer_->encode(sentence);
  std::fprintf(stderr, "kuiper: no tokenizer is loaded; pass token ids\n");
  return {};
}

}  // namespace model
