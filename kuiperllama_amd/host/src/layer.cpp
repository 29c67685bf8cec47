// Layers and the argmax sampler of the host API (the reference's
// source/op/{layer,matmul,rmsnorm,rope,mha,swiglu,add,embedding}.cpp and
// source/sampler/argmax_sampler.cpp), dispatching to the kDeviceHIP kernels.
#include <numeric>

#include "kuiper/kernels.h"
#include "kuiper/layer.h"
#include "kuiper_hip.h"

namespace op {

BaseLayer::BaseLayer(base::DeviceType device_type, LayerType layer_type, base::DataType data_type,
                     std::string layer_name)
    : layer_name_(std::move(layer_name)),
      layer_type_(layer_type),
      data_type_(data_type),
      device_type_(device_type) {}

base::Status BaseLayer::set_weight(int32_t, const tensor::Tensor&) {
  return base::error::FunctionNotImplement();
}

base::Status BaseLayer::set_weight(int32_t, const std::vector<int32_t>&, const void*,
                                   base::DeviceType) {
  return base::error::FunctionNotImplement();
}

Layer::Layer(base::DeviceType device_type, LayerType layer_type, std::string layer_name)
    : BaseLayer(device_type, layer_type, base::DataType::kDataTypeFp32, std::move(layer_name)) {}

base::Status Layer::init() { return base::error::Success(); }

base::Status Layer::forward() { return base::error::FunctionNotImplement(""); }

// Which property of a layer operand does not match what the layer expects
// ("" when everything matches): presence, device, element type, then shape.
static std::string operand_mismatch(const tensor::Tensor& t, base::DeviceType device_type,
                                    base::DataType data_type, const std::vector<int32_t>* dims) {
  if (t.is_empty()) return "operand holds no data";
  if (t.device_type() != device_type) return "operand lives on another device";
  if (t.data_type() != data_type) return "operand element type differs from the layer's";
  if (!dims) return "";
  const int32_t rank = static_cast<int32_t>(dims->size());
  if (t.dims_size() != rank)
    return "operand rank " + std::to_string(t.dims_size()) + ", expected " + std::to_string(rank);
  for (int32_t i = 0; i < rank; ++i) {
    if (t.get_dim(i) != (*dims)[i])
      return "operand extent " + std::to_string(t.get_dim(i)) + " on axis " + std::to_string(i) +
             ", expected " + std::to_string((*dims)[i]);
  }
  return "";
}

base::Status Layer::check_tensor(const tensor::Tensor& tensor, base::DeviceType device_type,
                                 base::DataType data_type) const {
  const std::string why = operand_mismatch(tensor, device_type, data_type, nullptr);
  return why.empty() ? base::error::Success() : base::error::InvalidArgument(why);
}

base::Status Layer::check_tensor_with_dim(const tensor::Tensor& tensor,
                                          base::DeviceType device_type, base::DataType data_type,
                                          const std::vector<int32_t>& dims) const {
  const std::string why = operand_mismatch(tensor, device_type, data_type, &dims);
  return why.empty() ? base::error::Success() : base::error::InvalidArgument(why);
}

base::Status Layer::check() const {
  return base::error::FunctionNotImplement(layer_name_ + " defines no operand check");
}

base::Status Layer::forward(const tensor::Tensor& input1, const tensor::Tensor& output1) {
  set_input(0, input1);
  set_output(0, output1);
  return forward();
}

base::Status Layer::forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                            const tensor::Tensor& output1) {
  set_input(0, input1);
  set_input(1, input2);
  set_output(0, output1);
  return forward();
}

base::Status Layer::forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                            const tensor::Tensor& input3, const tensor::Tensor& output1) {
  set_input(0, input1);
  set_input(1, input2);
  set_input(2, input3);
  set_output(0, output1);
  return forward();
}

base::Status Layer::forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                            const tensor::Tensor& input3, const tensor::Tensor& input4,
                            const tensor::Tensor& output1) {
  set_input(0, input1);
  set_input(1, input2);
  set_input(2, input3);
  set_input(3, input4);
  set_output(0, output1);
  return forward();
}

base::Status Layer::forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                            const tensor::Tensor& input3, const tensor::Tensor& input4,
                            const tensor::Tensor& input5, const tensor::Tensor& output1) {
  set_input(0, input1);
  set_input(1, input2);
  set_input(2, input3);
  set_input(3, input4);
  set_input(4, input5);
  set_output(0, output1);
  return forward();
}

void Layer::set_input(int32_t idx, const tensor::Tensor& input) {
  KUIPER_CHECK(idx >= 0 && idx < static_cast<int32_t>(inputs_.size()), "input index");
  inputs_[idx] = input;
}

void Layer::set_output(int32_t idx, const tensor::Tensor& output) {
  KUIPER_CHECK(idx >= 0 && idx < static_cast<int32_t>(outputs_.size()), "output index");
  outputs_[idx] = output;
}

const tensor::Tensor& Layer::get_input(int32_t idx) const {
  KUIPER_CHECK(idx >= 0 && idx < static_cast<int32_t>(inputs_.size()), "input index");
  return inputs_[idx];
}
tensor::Tensor& Layer::get_input(int32_t idx) {
  KUIPER_CHECK(idx >= 0 && idx < static_cast<int32_t>(inputs_.size()), "input index");
  return inputs_[idx];
}
const tensor::Tensor& Layer::get_output(int32_t idx) const {
  KUIPER_CHECK(idx >= 0 && idx < static_cast<int32_t>(outputs_.size()), "output index");
  return outputs_[idx];
}
tensor::Tensor& Layer::get_output(int32_t idx) {
  KUIPER_CHECK(idx >= 0 && idx < static_cast<int32_t>(outputs_.size()), "output index");
  return outputs_[idx];
}

void Layer::to_hip() {
  for (auto& t : inputs_)
    if (!t.is_empty()) t.to_hip(stream());
  for (auto& t : outputs_)
    if (!t.is_empty()) t.to_hip(stream());
}

void Layer::set_hip_config(std::shared_ptr<kernel::HipConfig> config) {
  if (config) hip_config_ = std::move(config);
}

// ---------------------------------------------------------------------------
LayerParam::LayerParam(base::DeviceType device_type, LayerType layer_type, bool is_quant_layer,
                       std::string layer_name)
    : Layer(device_type, layer_type, std::move(layer_name)), is_quant_layer_(is_quant_layer) {}

tensor::Tensor& LayerParam::get_weight(int32_t idx) {
  KUIPER_CHECK(idx >= 0 && idx < static_cast<int32_t>(weights_.size()), "weight index");
  return weights_[idx];
}
const tensor::Tensor& LayerParam::get_weight(int32_t idx) const {
  KUIPER_CHECK(idx >= 0 && idx < static_cast<int32_t>(weights_.size()), "weight index");
  return weights_[idx];
}

base::Status LayerParam::set_weight(int32_t idx, const tensor::Tensor& weight) {
  KUIPER_CHECK(idx >= 0 && idx < static_cast<int32_t>(weights_.size()), "weight index");
  KUIPER_CHECK(weight.data_type() == base::DataType::kDataTypeFp32, "weight must be fp32");
  if (!weight.is_empty())
    KUIPER_CHECK(weight.device_type() == device_type_, "weight on another device");
  weights_[idx] = weight;
  return base::error::Success();
}

base::Status LayerParam::set_weight(int32_t idx, const std::vector<int32_t>& dims,
                                    const void* weight_ptr, base::DeviceType device_type) {
  KUIPER_CHECK(idx >= 0 && idx < static_cast<int32_t>(weights_.size()), "weight index");
  KUIPER_CHECK(weight_ptr != nullptr, "null weight pointer");
  const size_t n = std::accumulate(dims.begin(), dims.end(), size_t(1),
                                   [](size_t a, int32_t b) { return a * static_cast<size_t>(b); });
  void* p = const_cast<void*>(weight_ptr);
  if (!is_quant_layer_) {
    auto buffer = std::make_shared<base::Buffer>(n * sizeof(float), nullptr, p, true);
    if (device_type != base::DeviceType::kDeviceUnknown) buffer->set_device_type(device_type);
    tensor::Tensor weight(base::DataType::kDataTypeFp32, dims);
    weight.set_device_type(device_type);
    KUIPER_CHECK(weight.assign(buffer), "weight assign");
    weights_[idx] = weight;
  } else {
    auto buffer = std::make_shared<base::Buffer>(n, nullptr, p, true);
    if (device_type != base::DeviceType::kDeviceUnknown) buffer->set_device_type(device_type);
    tensor::Tensor weight(base::DataType::kDataTypeInt8, dims);
    KUIPER_CHECK(weight.assign(buffer), "weight assign");
    weights_[idx] = weight;
    KUIPER_CHECK(group_size_ > 0 && n % group_size_ == 0, "weight size not a multiple of group");
    const int32_t scale_nums = static_cast<int32_t>(n / group_size_);
    scales_ = tensor::Tensor(base::DataType::kDataTypeFp32, scale_nums, false, nullptr,
                             static_cast<int8_t*>(p) + n);
    scales_.set_device_type(device_type);
  }
  return base::error::Success();
}

void LayerParam::set_scales(const tensor::Tensor& scales) {
  KUIPER_CHECK(!scales.is_empty(), "empty scales");
  scales_ = scales;
}

int32_t LayerParam::get_scale_num() const {
  KUIPER_CHECK(!scales_.is_empty(), "no scales");
  return static_cast<int32_t>(scales_.size());
}

void LayerParam::to_hip() {
  Layer::to_hip();
  for (auto& w : weights_)
    if (!w.is_empty()) w.to_hip(stream());
  if (!scales_.is_empty()) scales_.to_hip(stream());
}

// ---------------------------------------------------------------------------
MatmulLayer::MatmulLayer(base::DeviceType device_type, int32_t dim0, int32_t dim1,
                         bool is_quant_layer, bool has_bias)
    : LayerParam(device_type, LayerType::kLayerMatmul, is_quant_layer, "Matmul"),
      dim0_(dim0),
      dim1_(dim1),
      has_bias_(has_bias) {
  reset_input_size(1);
  reset_output_size(1);
  reset_weight_size(1);
  if (has_bias_) bias_.resize(1);
}

base::Status MatmulLayer::check() const {
  base::Status s = check_tensor_with_dim(get_input(0), device_type_, data_type_, {dim1_});
  if (!s) return s;
  if (!is_quant_layer_) {
    s = check_tensor_with_dim(get_weight(0), device_type_, data_type_, {dim0_, dim1_});
  } else {
    s = check_tensor_with_dim(get_weight(0), device_type_, base::DataType::kDataTypeInt8,
                              {dim0_, dim1_});
    if (s) s = check_tensor(scales_, device_type_, base::DataType::kDataTypeFp32);
  }
  if (!s) return s;
  return check_tensor_with_dim(get_output(0), device_type_, data_type_, {dim0_});
}

base::Status MatmulLayer::forward() {
  base::Status s = check();
  if (!s) return s;
  if (is_quant_layer_) {
    kernel::get_matmul_kernel_quant8(device_type_)(get_input(0), get_weight(0), get_output(0),
                                                   group_size_, scales_, hip_config_.get());
  } else {
    kernel::get_matmul_kernel(device_type_)(get_input(0), get_weight(0), get_output(0), 1.f,
                                            hip_config_.get());
  }
  if (has_bias_)
    kernel::get_add_kernel(device_type_)(get_output(0), get_bias(0), get_output(0), stream());
  return base::error::Success();
}

base::Status MatmulLayer::set_bias(int32_t idx, int32_t& dim, const void* bias_ptr,
                                   base::DeviceType device_type) {
  KUIPER_CHECK(idx >= 0 && idx < static_cast<int32_t>(bias_.size()), "bias index");
  KUIPER_CHECK(bias_ptr != nullptr, "null bias pointer");
  auto buffer = std::make_shared<base::Buffer>(static_cast<size_t>(dim) * sizeof(float), nullptr,
                                               const_cast<void*>(bias_ptr), true);
  if (device_type != base::DeviceType::kDeviceUnknown) buffer->set_device_type(device_type);
  tensor::Tensor bias(base::DataType::kDataTypeFp32, dim);
  bias.set_device_type(device_type);
  KUIPER_CHECK(bias.assign(buffer), "bias assign");
  bias_[idx] = bias;
  return base::error::Success();
}

tensor::Tensor& MatmulLayer::get_bias(int32_t idx) {
  KUIPER_CHECK(idx >= 0 && idx < static_cast<int32_t>(bias_.size()), "bias index");
  return bias_[idx];
}
const tensor::Tensor& MatmulLayer::get_bias(int32_t idx) const {
  KUIPER_CHECK(idx >= 0 && idx < static_cast<int32_t>(bias_.size()), "bias index");
  return bias_[idx];
}

void MatmulLayer::to_hip() {
  LayerParam::to_hip();
  for (auto& b : bias_)
    if (!b.is_empty()) b.to_hip(stream());
}

// ---------------------------------------------------------------------------
RmsNormLayer::RmsNormLayer(base::DeviceType device_type, int32_t dim)
    : LayerParam(device_type, LayerType::kLayerRMSNorm, false, "RMSNorm"), dim_(dim) {
  reset_input_size(1);
  reset_output_size(1);
  reset_weight_size(1);
}

base::Status RmsNormLayer::check() const {
  const tensor::Tensor& in = get_input(0);
  base::Status s = check_tensor(in, device_type_, data_type_);
  if (!s) return s;
  if (in.size() % dim_ != 0)
    return base::error::InvalidArgument("The input size is not a multiple of the norm width.");
  s = check_tensor_with_dim(get_weight(0), device_type_, data_type_, {dim_});
  if (!s) return s;
  s = check_tensor(get_output(0), device_type_, data_type_);
  if (!s) return s;
  if (get_output(0).size() != in.size())
    return base::error::InvalidArgument("The output size differs from the input size.");
  return base::error::Success();
}

base::Status RmsNormLayer::forward() {
  base::Status s = check();
  if (!s) return s;
  if (get_input(0).size() == static_cast<size_t>(dim_))
    kernel::get_rmsnorm_kernel(device_type_)(get_input(0), get_weight(0), get_output(0), stream());
  else
    kernel::get_rmsnorm_dim_kernel(device_type_)(get_input(0), get_weight(0), get_output(0), dim_,
                                                 stream());
  return base::error::Success();
}

// ---------------------------------------------------------------------------
RoPELayer::RoPELayer(base::DeviceType device_type, int32_t dim, int32_t kv_dim, int32_t head_size)
    : Layer(device_type, LayerType::kLayerRoPe, "RoPe"),
      dim_(dim),
      kv_dim_(kv_dim),
      head_size_(head_size) {
  reset_input_size(5);
  reset_output_size(1);
}

base::Status RoPELayer::check() const {
  base::Status s = check_tensor_with_dim(get_input(2), base::DeviceType::kDeviceCPU,
                                         base::DataType::kDataTypeInt32, {1});
  if (!s) return s;
  s = check_tensor_with_dim(get_input(1), device_type_, data_type_, {kv_dim_});
  if (!s) return s;
  s = check_tensor_with_dim(get_input(0), device_type_, data_type_, {dim_});
  if (!s) return s;
  s = check_tensor(get_input(3), device_type_, data_type_);
  if (!s) return s;
  return check_tensor(get_input(4), device_type_, data_type_);
}

base::Status RoPELayer::forward() {
  base::Status s = check();
  if (!s) return s;
  kernel::get_rope_kernel(device_type_)(dim_, kv_dim_, head_size_, get_input(0), get_input(1),
                                        get_input(2), get_input(3), get_input(4), stream());
  return base::error::Success();
}

// ---------------------------------------------------------------------------
MultiHeadAttention::MultiHeadAttention(base::DeviceType device_type, int32_t layer_index,
                                       int32_t kv_mul, int32_t kv_dim, int32_t seq_len,
                                       int32_t head_num, int32_t head_size)
    : Layer(device_type, LayerType::kLayerMHA, "MultiHead"),
      layer_index_(layer_index),
      kv_mul_(kv_mul),
      kv_dim_(kv_dim),
      seq_len_(seq_len),
      head_num_(head_num),
      head_size_(head_size) {
  reset_input_size(4);
  reset_output_size(1);
}

base::Status MultiHeadAttention::check() const {
  for (int32_t i = 0; i < 4; ++i) {
    base::Status s = check_tensor(get_input(i), device_type_, data_type_);
    if (!s) return s;
  }
  return check_tensor(get_output(0), device_type_, data_type_);
}

base::Status MultiHeadAttention::forward() {
  base::Status s = check();
  if (!s) return s;
  kernel::get_mha_kernel(device_type_)(pos_, head_num_, layer_index_, seq_len_, kv_dim_, kv_mul_,
                                       head_size_, get_output(0), get_input(0), get_input(1),
                                       get_input(2), get_input(3), device_type_,
                                       hip_config_.get());
  return base::error::Success();
}

// ---------------------------------------------------------------------------
SwiGLULayer::SwiGLULayer(base::DeviceType device_type, int32_t hidden_dim)
    : Layer(device_type, LayerType::kLayerSwiGLU, "SwiGLU"), hidden_dim_(hidden_dim) {
  reset_input_size(2);
  reset_output_size(1);
}

base::Status SwiGLULayer::check() const {
  base::Status s = check_tensor_with_dim(get_input(0), device_type_, data_type_, {hidden_dim_});
  if (!s) return s;
  s = check_tensor_with_dim(get_input(1), device_type_, data_type_, {hidden_dim_});
  if (!s) return s;
  return check_tensor_with_dim(get_output(0), device_type_, data_type_, {hidden_dim_});
}

base::Status SwiGLULayer::forward() {
  base::Status s = check();
  if (!s) return s;
  kernel::get_swiglu_kernel(device_type_)(get_input(0), get_input(1), get_output(0), stream());
  return base::error::Success();
}

// ---------------------------------------------------------------------------
VecAddLayer::VecAddLayer(base::DeviceType device_type)
    : Layer(device_type, LayerType::kLayerAdd, "Add") {
  reset_input_size(2);
  reset_output_size(1);
}

base::Status VecAddLayer::check() const {
  const int32_t n = static_cast<int32_t>(get_input(0).size());
  base::Status s = check_tensor_with_dim(get_input(0), device_type_, data_type_, {n});
  if (!s) return s;
  s = check_tensor_with_dim(get_input(1), device_type_, data_type_, {n});
  if (!s) return s;
  return check_tensor_with_dim(get_output(0), device_type_, data_type_, {n});
}

base::Status VecAddLayer::forward() {
  base::Status s = check();
  if (!s) return s;
  kernel::get_add_kernel(device_type_)(get_input(0), get_input(1), get_output(0), stream());
  return base::error::Success();
}

// ---------------------------------------------------------------------------
EmbeddingLayer::EmbeddingLayer(base::DeviceType device_type, int32_t dim, int32_t seq_len,
                               int32_t vocab_size)
    : LayerParam(device_type, LayerType::kLayerEmbedding, false, "Embedding"),
      dim_(dim),
      seq_len_(seq_len),
      vocab_size_(vocab_size) {
  reset_input_size(2);
  reset_output_size(1);
  reset_weight_size(1);
}

base::Status EmbeddingLayer::check() const {
  const tensor::Tensor& input = get_input(0);
  const int32_t token_size = static_cast<int32_t>(get_input(1).size());
  if (token_size > static_cast<int32_t>(input.size()))
    return base::error::InvalidArgument("more token ids than the layer's sequence length");
  base::Status s = check_tensor_with_dim(input, base::DeviceType::kDeviceCPU,
                                         base::DataType::kDataTypeInt32, {token_size});
  if (!s) return s;
  s = check_tensor_with_dim(get_weight(0), device_type_, data_type_, {vocab_size_, dim_});
  if (!s) return s;
  return check_tensor_with_dim(get_output(0), device_type_, data_type_, {token_size, dim_});
}

base::Status EmbeddingLayer::forward() {
  base::Status s = check();
  if (!s) return s;
  kernel::get_emb_kernel(device_type_)(get_input(0), get_weight(0), get_output(0), vocab_size_,
                                       stream());
  return base::error::Success();
}

}  // namespace op

// ---------------------------------------------------------------------------
namespace sampler {

ArgmaxSampler::~ArgmaxSampler() {
  if (workspace_) kl_free(workspace_);
}

size_t ArgmaxSampler::sample(const float* logits, size_t size, void* stream) {
  KUIPER_CHECK(logits != nullptr && size > 0 && size <= 0x7fffffffu, "bad logits");
  if (device_type_ == base::DeviceType::kDeviceCPU) {
    size_t best = 0;  // std::max_element: the first maximum
    for (size_t i = 1; i < size; ++i)
      if (logits[i] > logits[best]) best = i;
    return best;
  }
  KUIPER_CHECK(device_type_ == base::DeviceType::kDeviceHIP, "unsupported sampler device");
  size_t need = 0;
  KUIPER_CHECK(kl_argmax_workspace_size(static_cast<int>(size), &need) == KL_OK, "argmax size");
  const size_t total = need + 256;  // the index lives after the partials
  if (total > workspace_bytes_) {
    if (workspace_) kl_free(workspace_);
    workspace_ = nullptr;
    KUIPER_CHECK(kl_malloc(&workspace_, total) == KL_OK, "argmax workspace allocation");
    KUIPER_CHECK(kl_memset_zero(workspace_, total, stream) == KL_OK, "argmax workspace zero");
    workspace_bytes_ = total;
  }
  int32_t* d_index = reinterpret_cast<int32_t*>(static_cast<char*>(workspace_) + workspace_bytes_ - 256);
  int rc = kl_argmax(logits, static_cast<int>(size), d_index, workspace_, workspace_bytes_ - 256,
                     stream);
  KUIPER_CHECK(rc == KL_OK, std::string("kl_argmax: ") + kl_error_string(rc));
  int32_t idx = -1;
  rc = kl_memcpy_d2h(&idx, d_index, sizeof(idx), stream);
  KUIPER_CHECK(rc == KL_OK, "argmax copy");
  KUIPER_CHECK(kl_stream_sync(stream) == KL_OK, "argmax sync");
  return static_cast<size_t>(idx);
}

}  // namespace sampler
