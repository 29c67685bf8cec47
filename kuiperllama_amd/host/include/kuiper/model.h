// Models of the host API: Model (the reference's include/model/model.h:14-94)
// and LLama2Model / Qwen2Model / Qwen3Model (include/model/llama3.h:33-74,
// qwen2.h:42-87, qwen3.h:48-89).  init(kDeviceHIP) mmaps a reference-format
// .bin file, wraps the weights as layers and moves them to the device;
// predict() runs the reference's layer-by-layer forward on the HIP kernels.
// set_fused(true) runs predict() on the fused decode engine of the C ABI
// (kl_engine_*) instead, from the same mapped file.
//
// Differences from the reference, by design:
//  * the model family (RoPE pairing and theta, RMSNorm eps, Qwen2 bias, Qwen3
//    q/k norm, header size) is a constructor argument instead of a build flag;
//  * the tokenizer is optional: with an empty token_path prompts are token
//    ids (encode/decode report that no tokenizer is loaded); with one, the
//    family picks the layer (SentencePiece for kEncodeSpe; byte-level BPE
//    with the Qwen special tokens for the Qwen families, the Llama-3 ones
//    otherwise) and the model's vocabulary size stays the image's;
//  * kDeviceCPU is refused: the CPU kernels are the reference's own.
#pragma once
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "kuiper/encode.h"
#include "kuiper/hip_config.h"
#include "kuiper/kernels.h"
#include "kuiper/layer.h"
#include "kuiper/tensor.h"

struct kl_engine;

namespace model {

enum class ModelFamily : int32_t {
  kLlama2 = 0,  // interleaved RoPE, theta 1e4, eps 1e-5 (no build flag)
  kLlama3 = 1,  // rotate-half RoPE, theta 5e5, eps 1e-5 (LLAMA3_SUPPORT)
  kQwen2 = 2,   // rotate-half, theta 1e6, eps 1e-6, q/k/v bias (QWEN2_SUPPORT)
  kQwen3 = 3,   // rotate-half, theta 1e6, eps 1e-6, per-head q/k RMSNorm (QWEN3_SUPPORT)
};

// The .bin header (include/model/config.h:4-15): 7 int32, plus the group size
// for int8 images; Qwen3 images carry 8 int32 {q_dim, dim, layers, heads,
// kv_heads, vocab, seq_len, ffn_dim}.
struct ModelConfig {
  int32_t dim = 0;
  int32_t hidden_dim = 0;
  int32_t layer_num = 0;
  int32_t head_num = 0;
  int32_t kv_head_num = 0;
  int32_t vocab_size = 0;
  int32_t seq_len = 0;
};

// Derived sizes (model/model.cpp:113-141).  dim_ is the model width,
// q_dim_ = head_num * head_size (equal to dim_ except Qwen3), hidden_dim_ the
// FFN width.
struct TransformerConfig {
  int32_t kv_dim_ = 0;
  int32_t kv_mul_ = 0;
  int32_t head_size_ = 0;
  int32_t vocab_size_ = 0;
  int32_t dim_ = 0;
  int32_t q_dim_ = 0;
  int32_t hidden_dim_ = 0;
  int32_t layer_num_ = 0;
  int32_t head_num_ = 0;
  int32_t kv_head_num_ = 0;
  int32_t seq_len_ = 0;
  bool is_shared_weight_ = false;
};

// A read-only mapping of the model file (model/raw_model_data.cpp).
struct RawModelData {
  int32_t fd = -1;
  size_t file_size = 0;
  void* data = nullptr;
  const int8_t* weight_data = nullptr;  // first byte after the header
  ~RawModelData();
};

struct DecoderLayers {
  std::shared_ptr<op::Layer> add_layer_, rope_layer_, swiglu_layer_, mha_layer_;
  std::vector<std::shared_ptr<op::Layer>> wq_layers_, wk_layers_, wv_layers_, wo_layers_;
  std::vector<std::shared_ptr<op::Layer>> w1_layers_, w2_layers_, w3_layers_;
  // 0..L-1 attention norms, L..2L-1 FFN norms, 2L the final norm; Qwen3:
  // 2L+1..3L q norms, 3L+1..4L k norms.
  std::vector<std::shared_ptr<op::Layer>> rmsnorm_layers_;
  std::shared_ptr<op::Layer> cls_layer_, embedding_layer_;
  void to_hip(const std::shared_ptr<kernel::HipConfig>& config);
};

// One operation's device time over the profiled predict() calls
// (model/qwen2.h:13-18).
struct OpProfileStat {
  std::string op_name;
  double total_ms = 0.0;
  int64_t calls = 0;
  double avg_ms = 0.0;
};

// The model interface (include/model/model.h:14-94): init, predict, forward,
// embedding, post_processing and the layer/buffer factories are pure virtual,
// implemented by each family's class; the file reading, buffers, tokenizer
// and the fused engine are shared.
class Model {
 public:
  explicit Model(base::TokenizerType tokenizer_type, base::ModelType model_type,
                 std::string token_path, std::string model_path, bool is_quant_model,
                 ModelFamily family);
  virtual ~Model();

  virtual base::Status init(base::DeviceType device_type) = 0;
  // One token: forward() then, unless is_prompt, greedy sampling into next
  // (-1 for prompt positions), as llama3.cpp:641-649.
  virtual base::Status predict(const tensor::Tensor& input, const tensor::Tensor& pos_tensor,
                               bool is_prompt, int& next) const = 0;
  virtual base::Status forward(const tensor::Tensor& input, const tensor::Tensor& pos_tensor,
                               int& next) const = 0;

  base::ModelType model_type() const { return model_type_; }
  ModelFamily family() const { return family_; }
  const std::string& token_path() const { return token_path_; }
  const std::string& model_path() const { return model_path_; }
  const TransformerConfig& config() const { return *config_; }
  virtual tensor::Tensor& get_buffer(ModelBufferType buffer_idx);
  virtual const tensor::Tensor& get_buffer(ModelBufferType buffer_idx) const;

  virtual bool is_sentence_ending(int32_t token_idx) const;
  virtual std::string decode(int32_t token_idx) const;
  virtual std::string decode(std::vector<int32_t> token_idxs) const;
  virtual std::vector<int32_t> encode(const std::string& sentence) const;

  // K and V cache rows of (layer, position) as device tensors [kv_dim].
  virtual std::pair<tensor::Tensor, tensor::Tensor> slice_kv_cache(int32_t layer_idx,
                                                                   int32_t token_pos) const;
  // Embeds tokens (all at once) into kInputEmbeddings.
  virtual op::EmbeddingOutput embedding(const std::vector<int>& tokens) const = 0;
  // The residual-stream input of a step: row pos of the prompt embeddings
  // (is_prompt) or row 0 (the single decoded token), as model.cpp:240-265.
  virtual tensor::Tensor fill_input(const tensor::Tensor& pos_tensor,
                                    const op::EmbeddingOutput& embedding_output,
                                    bool is_prompt) const;

  // Fused decode engine (one persistent launch per token); predict() uses it
  // when enabled.  The engine is created on first use from the mapped file.
  base::Status set_fused(bool enable);
  bool is_fused() const { return fused_; }
  // The greedy loop of demo/main.cpp:5-47: P prompt tokens, then n_new
  // sampled tokens written to out (fused: entirely on the device; layered:
  // through the virtual embedding(), fill_input() and predict()).
  base::Status generate(const std::vector<int32_t>& prompt, int32_t n_new,
                        std::vector<int32_t>& out) const;
  // Fused only: the whole prompt in one batched pass (kl_engine_prefill);
  // next receives the greedy token after the prompt and kForwardOutput the
  // logits of its last position.  Decoding continues with predict() at
  // position prompt.size().  generate() uses it when set_prefill(true).
  base::Status prefill(const std::vector<int32_t>& prompt, int& next) const;
  base::Status set_prefill(bool enable);
  // More end-of-sequence ids for is_sentence_ending(), besides the
  // tokenizer's (encode.cpp); the only ones when no tokenizer is loaded.
  void set_eos_tokens(std::vector<int32_t> ids) { eos_tokens_ = std::move(ids); }
  std::shared_ptr<kernel::HipConfig> hip_config() const { return hip_config_; }
  // Per-operation profile of predict() (qwen2.cpp:20-57, :820-822), timed on
  // the device: HIP events on the model's stream bracket each operation (the
  // reference times the host-side launch).  Names as the reference's
  // ("attn.rmsnorm", "attn.wq", ..., "ffn.w2", "output.cls", "sampler.argmax",
  // plus "input.embedding" for embedding()); the fused step is one
  // "fused.step" per token and prefill() one "prefill.batched".  Off until
  // reset_profile_stats() is called; each profiled call waits for the device.
  void reset_profile_stats() const;
  std::vector<OpProfileStat> get_profile_stats() const;

 protected:
  virtual base::Status insert_buffer(ModelBufferType buffer_idx, const tensor::Tensor& tensor);
  virtual base::Status read_model_file();
  virtual base::Status create_encode_layer();
  // model.cpp:113-141: the header's sizes into config_; `extra` is the
  // eighth header int of layouts that have one (int8: the group size, read
  // before this call; Qwen3: the FFN width).
  virtual base::Status generate_model_infos(const ModelConfig& config, int32_t extra);
  virtual int32_t post_processing(const tensor::Tensor& pos, bool is_prompt) const = 0;
  virtual void init_mem() = 0;
  virtual base::Status create_layers() = 0;
  virtual void create_param_layers() = 0;
  virtual void create_nonparam_layers() = 0;
  virtual void create_param_quant_layers() = 0;
  // Runs fn, bracketed by profile events on `stream` (default: the model's)
  // when profiling is on.
  template <class Fn>
  void profiled(const char* name, Fn&& fn, void* stream = nullptr) const;
  void resolve_profile() const;

  int32_t group_size_ = 1;
  bool is_quant_model_ = false;
  ModelFamily family_ = ModelFamily::kLlama2;
  std::unique_ptr<TransformerConfig> config_;
  std::string token_path_;
  std::string model_path_;
  std::map<ModelBufferType, tensor::Tensor> buffers_;
  std::unique_ptr<sampler::Sampler> sampler_;
  std::shared_ptr<RawModelData> raw_model_data_;
  base::DeviceType device_type_ = base::DeviceType::kDeviceUnknown;
  base::ModelType model_type_ = base::ModelType::kModelTypeUnknown;
  base::TokenizerType tokenizer_type_ = base::TokenizerType::kEncodeUnknown;
  std::shared_ptr<kernel::HipConfig> hip_config_;
  std::unique_ptr<DecoderLayers> layers_;
  bool fused_ = false;
  bool prefill_ = false;
  std::vector<int32_t> eos_tokens_;
  std::unique_ptr<op::EncodeLayerBase> encode_layer_;
  kl_engine* engine_ = nullptr;
  struct ProfileRecord {
    const char* name;
    void* start;
    void* stop;
  };
  mutable bool profiling_ = false;
  mutable std::map<std::string, std::pair<double, int64_t>> profile_;
  mutable std::vector<ProfileRecord> profile_pending_;
  mutable std::vector<void*> profile_events_;  // free events for reuse
  mutable std::vector<void*> profile_all_events_;
};

// Llama2 (default) and Llama3 (family kLlama3) checkpoints: the decoder of
// include/model/llama3.h:33-74 (llama3.cpp), layer by layer on the HIP
// kernels.  Its step stages are virtual so a family can change one.
class LLama2Model : public Model {
 public:
  explicit LLama2Model(base::TokenizerType tokenizer_type, std::string token_path,
                       std::string model_path, bool is_quant_model,
                       ModelFamily family = ModelFamily::kLlama2);

  base::Status init(base::DeviceType device_type) override;
  base::Status predict(const tensor::Tensor& input, const tensor::Tensor& pos_tensor,
                       bool is_prompt, int& next) const override;
  base::Status forward(const tensor::Tensor& input, const tensor::Tensor& pos_tensor,
                       int& next) const override;
  op::EmbeddingOutput embedding(const std::vector<int>& tokens) const override;

 protected:
  int32_t post_processing(const tensor::Tensor& pos, bool is_prompt) const override;
  void init_mem() override;
  base::Status create_layers() override;
  void create_param_layers() override;
  void create_nonparam_layers() override;
  void create_param_quant_layers() override;
  // The fp32 walk of llama3.cpp:289-422 (with_bias: qwen2.cpp:348-485, a
  // bias vector after each of wq, wk, wv).
  void create_param_layers_fp32(bool with_bias);
  // Bytes the fp32 layout needs after the header (create_layers checks the file).
  virtual size_t fp32_weight_bytes() const;

  virtual void attention_rms(int32_t layer_idx, const tensor::Tensor& input) const;
  virtual void attention_qkv(int32_t layer_idx, const tensor::Tensor& pos_tensor) const;
  virtual void attention_mha(int32_t layer_idx, const tensor::Tensor& pos_tensor) const;
  virtual void feed_forward(int32_t layer_idx, const tensor::Tensor& input) const;
  virtual void cls_logits(const tensor::Tensor& input) const;
};

// Qwen2 / Qwen2.5 (include/model/qwen2.h:42-87): the Llama decoder with
// q/k/v biases in the fp32 layout (the int8 layout has none, qwen2.cpp:242-346).
class Qwen2Model : public LLama2Model {
 public:
  explicit Qwen2Model(base::TokenizerType tokenizer_type, std::string token_path,
                      std::string model_path, bool is_quant_model);

 protected:
  void create_param_layers() override;
  size_t fp32_weight_bytes() const override;
};

// Qwen3 (include/model/qwen3.h:48-89): an 8-int header {q_dim, dim, ...,
// ffn_dim}, norms first and a separate lm_head in the file, q_dim != dim, and
// a per-head q/k RMSNorm before RoPE.  fp32 only.
class Qwen3Model : public LLama2Model {
 public:
  explicit Qwen3Model(base::TokenizerType tokenizer_type, std::string token_path,
                      std::string model_path, bool is_quant_model);
  base::Status init(base::DeviceType device_type) override;

 protected:
  base::Status generate_model_infos(const ModelConfig& config, int32_t extra) override;
  void create_param_layers() override;
  size_t fp32_weight_bytes() const override;
  void attention_qkv(int32_t layer_idx, const tensor::Tensor& pos_tensor) const override;
};

}  // namespace model
