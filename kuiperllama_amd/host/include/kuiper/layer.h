// Layers of the host API: BaseLayer / Layer / LayerParam (the reference's
// include/op/layer.h:11-188) and the compute layers of the decode step
// (include/op/{matmul,rmsnorm,rope,mha,swiglu,add,embedding}.h).  forward()
// checks the tensors and dispatches through kernel::get_*_kernel(device_type_).
#pragma once
#include <memory>
#include <string>
#include <vector>

#include "kuiper/base.h"
#include "kuiper/hip_config.h"
#include "kuiper/tensor.h"

namespace op {

enum class LayerType : uint8_t {
  kLayerUnknown = 0,
  kLayerLinear = 1,
  kLayerEncode = 2,
  kLayerEmbedding = 3,
  kLayerRMSNorm = 4,
  kLayerMatmul = 5,
  kLayerRoPe = 6,
  kLayerMHA = 7,
  kLayerSoftmax = 8,
  kLayerAdd = 9,
  kLayerSwiGLU = 10,
};

class BaseLayer {
 public:
  explicit BaseLayer(base::DeviceType device_type, LayerType layer_type, base::DataType data_type,
                     std::string layer_name = "");
  virtual ~BaseLayer() = default;
  base::DataType data_type() const { return data_type_; }
  LayerType layer_type() const { return layer_type_; }
  virtual base::Status init() = 0;
  virtual base::Status forward() = 0;
  virtual base::Status forward(const tensor::Tensor& input1, const tensor::Tensor& output1) = 0;
  virtual base::Status forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                               const tensor::Tensor& output1) = 0;
  virtual base::Status forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                               const tensor::Tensor& input3, const tensor::Tensor& output1) = 0;
  virtual base::Status forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                               const tensor::Tensor& input3, const tensor::Tensor& input4,
                               const tensor::Tensor& output1) = 0;
  virtual base::Status forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                               const tensor::Tensor& input3, const tensor::Tensor& input4,
                               const tensor::Tensor& input5, const tensor::Tensor& output1) = 0;
  virtual void set_input(int32_t idx, const tensor::Tensor& input) = 0;
  virtual void set_output(int32_t idx, const tensor::Tensor& output) = 0;
  virtual size_t input_size() const = 0;
  virtual size_t output_size() const = 0;
  virtual base::Status check() const = 0;
  virtual tensor::Tensor& get_input(int32_t idx) = 0;
  virtual tensor::Tensor& get_output(int32_t idx) = 0;
  virtual const tensor::Tensor& get_input(int32_t idx) const = 0;
  virtual const tensor::Tensor& get_output(int32_t idx) const = 0;
  virtual base::Status set_weight(int32_t idx, const tensor::Tensor& weight);
  virtual base::Status set_weight(int32_t idx, const std::vector<int32_t>& dims,
                                  const void* weight_ptr,
                                  base::DeviceType device_type = base::DeviceType::kDeviceUnknown);
  const std::string& get_layer_name() const { return layer_name_; }
  void set_layer_name(const std::string& layer_name) { layer_name_ = layer_name; }
  base::DeviceType device_type() const { return device_type_; }
  void set_device_type(base::DeviceType device_type) { device_type_ = device_type; }

 protected:
  std::string layer_name_;
  LayerType layer_type_ = LayerType::kLayerUnknown;
  base::DataType data_type_ = base::DataType::kDataTypeUnknown;
  base::DeviceType device_type_ = base::DeviceType::kDeviceUnknown;
};

class Layer : public BaseLayer {
 public:
  explicit Layer(base::DeviceType device_type, LayerType layer_type, std::string layer_name = "");
  base::Status init() override;
  base::Status check_tensor(const tensor::Tensor& tensor, base::DeviceType device_type,
                            base::DataType data_type) const;
  // Checks emptiness, device, data type and, in order, each dimension.
  base::Status check_tensor_with_dim(const tensor::Tensor& tensor, base::DeviceType device_type,
                                     base::DataType data_type,
                                     const std::vector<int32_t>& dims) const;
  base::Status check() const override;
  base::Status forward() override;
  base::Status forward(const tensor::Tensor& input1, const tensor::Tensor& output1) override;
  base::Status forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                       const tensor::Tensor& output1) override;
  base::Status forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                       const tensor::Tensor& input3, const tensor::Tensor& output1) override;
  base::Status forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                       const tensor::Tensor& input3, const tensor::Tensor& input4,
                       const tensor::Tensor& output1) override;
  base::Status forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                       const tensor::Tensor& input3, const tensor::Tensor& input4,
                       const tensor::Tensor& input5, const tensor::Tensor& output1) override;
  void set_input(int32_t idx, const tensor::Tensor& input) override;
  void set_output(int32_t idx, const tensor::Tensor& output) override;
  const tensor::Tensor& get_input(int32_t idx) const override;
  const tensor::Tensor& get_output(int32_t idx) const override;
  tensor::Tensor& get_input(int32_t idx) override;
  tensor::Tensor& get_output(int32_t idx) override;
  size_t input_size() const override { return inputs_.size(); }
  size_t output_size() const override { return outputs_.size(); }
  void reset_input_size(size_t size) { inputs_.resize(size); }
  void reset_output_size(size_t size) { outputs_.resize(size); }
  // Moves the layer's tensors to the HIP device (the reference's to_cuda()).
  virtual void to_hip();
  void set_hip_config(std::shared_ptr<kernel::HipConfig> config);
  std::shared_ptr<kernel::HipConfig> hip_config() const { return hip_config_; }

 protected:
  void* stream() const { return hip_config_ ? hip_config_->stream : nullptr; }
  std::vector<tensor::Tensor> inputs_;
  std::vector<tensor::Tensor> outputs_;
  std::shared_ptr<kernel::HipConfig> hip_config_;
};

class LayerParam : public Layer {
 public:
  explicit LayerParam(base::DeviceType device_type, LayerType layer_type,
                      bool is_quant_layer = false, std::string layer_name = "");
  size_t weight_size() const { return weights_.size(); }
  void reset_weight_size(size_t size) { weights_.resize(size); }
  tensor::Tensor& get_weight(int32_t idx);
  const tensor::Tensor& get_weight(int32_t idx) const;
  void to_hip() override;
  base::Status set_weight(int32_t idx, const tensor::Tensor& weight) override;
  // Wraps external memory (e.g. the mmap'd model file) as weight idx; for a
  // quantised layer the fp32 scales follow the int8 weights in memory
  // (layer.cpp:184-219 of the reference).
  base::Status set_weight(int32_t idx, const std::vector<int32_t>& dims, const void* weight_ptr,
                          base::DeviceType device_type = base::DeviceType::kDeviceUnknown) override;
  void set_scales(const tensor::Tensor& scales);
  void set_group_size(int32_t group_size) { group_size_ = group_size; }
  int32_t get_scale_num() const;

 protected:
  int32_t group_size_ = 0;
  bool is_quant_layer_ = false;
  tensor::Tensor scales_;
  std::vector<tensor::Tensor> weights_;
};

// y = W x (+ bias): W [dim0 x dim1] fp32, or int8 with scales (op/matmul.cpp).
class MatmulLayer : public LayerParam {
 public:
  explicit MatmulLayer(base::DeviceType device_type, int32_t dim0, int32_t dim1,
                       bool is_quant_layer = false, bool has_bias = false);
  base::Status check() const override;
  base::Status forward() override;
  using Layer::forward;
  base::Status set_bias(int32_t idx, int32_t& dim, const void* bias_ptr,
                        base::DeviceType device_type);
  tensor::Tensor& get_bias(int32_t idx);
  const tensor::Tensor& get_bias(int32_t idx) const;
  void to_hip() override;

 private:
  int32_t dim0_ = 0;
  int32_t dim1_ = 0;
  bool has_bias_ = false;
  std::vector<tensor::Tensor> bias_;
};

// RMSNorm of a vector [dim], or of each row of [rows x dim] (op/rmsnorm.cpp).
class RmsNormLayer : public LayerParam {
 public:
  explicit RmsNormLayer(base::DeviceType device_type, int32_t dim);
  base::Status check() const override;
  base::Status forward() override;
  using Layer::forward;

 private:
  int32_t dim_ = 0;
};

// Inputs: q [dim], k [kv_dim], pos (CPU int32 [1]), sin, cos (op/rope.cpp).
class RoPELayer : public Layer {
 public:
  explicit RoPELayer(base::DeviceType device_type, int32_t dim, int32_t kv_dim, int32_t head_size);
  base::Status check() const override;
  base::Status forward() override;
  using Layer::forward;

 private:
  int32_t dim_ = 0;
  int32_t kv_dim_ = 0;
  int32_t head_size_ = 0;
};

// Inputs: query, score storage, key cache, value cache; output [dim] (op/mha.cpp).
class MultiHeadAttention : public Layer {
 public:
  explicit MultiHeadAttention(base::DeviceType device_type, int32_t layer_index, int32_t kv_mul,
                              int32_t kv_dim, int32_t seq_len, int32_t head_num,
                              int32_t head_size);
  base::Status check() const override;
  base::Status forward() override;
  using Layer::forward;
  void set_pos(int32_t pos) { pos_ = pos; }
  void set_layer_idx(int32_t layer_idx) { layer_index_ = layer_idx; }

 private:
  int32_t layer_index_ = 0;
  int32_t pos_ = 0;
  int32_t kv_mul_ = 0;
  int32_t kv_dim_ = 0;
  int32_t seq_len_ = 0;
  int32_t head_num_ = 0;
  int32_t head_size_ = 0;
};

// out = a * sigmoid(a) * b (op/swiglu.cpp).
class SwiGLULayer : public Layer {
 public:
  explicit SwiGLULayer(base::DeviceType device_type, int32_t hidden_dim);
  base::Status check() const override;
  base::Status forward() override;
  using Layer::forward;

 private:
  int32_t hidden_dim_ = 0;
};

// out = a + b (op/add.cpp).
class VecAddLayer : public Layer {
 public:
  explicit VecAddLayer(base::DeviceType device_type);
  base::Status check() const override;
  base::Status forward() override;
  using Layer::forward;
};

// Inputs: token ids (CPU int32 [n]), token count; output [n x dim] (op/embedding.cpp).
struct EmbeddingOutput {
  tensor::Tensor input_tokens;
  tensor::Tensor input_embeddings;
  tensor::Tensor input_token_num;
  explicit EmbeddingOutput(tensor::Tensor input_tokens, tensor::Tensor input_embeddings,
                           tensor::Tensor input_token_num)
      : input_tokens(std::move(input_tokens)),
        input_embeddings(std::move(input_embeddings)),
        input_token_num(std::move(input_token_num)) {}
};

class EmbeddingLayer : public LayerParam {
 public:
  explicit EmbeddingLayer(base::DeviceType device_type, int32_t dim, int32_t seq_len,
                          int32_t vocab_size);
  base::Status check() const override;
  base::Status forward() override;
  using Layer::forward;

 private:
  int32_t dim_ = 0;
  int32_t seq_len_ = 0;
  int32_t vocab_size_ = 0;
};

}  // namespace op

namespace sampler {
// include/sampler/sampler.h:6-14, argmax_sampler.h.
class Sampler {
 public:
  explicit Sampler(base::DeviceType device_type) : device_type_(device_type) {}
  virtual ~Sampler() = default;
  virtual size_t sample(const float* logits, size_t size, void* stream = nullptr) = 0;

 protected:
  base::DeviceType device_type_;
};

// Greedy sampling: the first index of the maximum (std::max_element).  On
// kDeviceHIP `logits` is device memory; the index comes back as 4 bytes.
class ArgmaxSampler : public Sampler {
 public:
  explicit ArgmaxSampler(base::DeviceType device_type) : Sampler(device_type) {}
  ~ArgmaxSampler() override;
  size_t sample(const float* logits, size_t size, void* stream) override;

 private:
  void* workspace_ = nullptr;  // device: argmax partials + the index
  size_t workspace_bytes_ = 0;
};
}  // namespace sampler
