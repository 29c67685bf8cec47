// kDeviceHIP kernel adapters: each unpacks the reference kernel signature
// (source/op/kernels/kernels_interface.h:6-47) into one call of the C ABI.  A
// failed call is fatal, as a failed CHECK inside the reference's kernels is.
#include <algorithm>
#include <cmath>
#include <string>

#include "kuiper/alloc.h"
#include "kuiper/kernels.h"
#include "kuiper_hip.h"

namespace kernel {

namespace {
KernelTraits g_traits;

void check_rc(int rc, const char* what) {
  if (rc != KL_OK) base::fatal(__FILE__, __LINE__, std::string(what) + ": " + kl_error_string(rc));
}

void require_hip(const tensor::Tensor& t, const char* name) {
  KUIPER_CHECK(!t.is_empty(), std::string(name) + " is empty");
  KUIPER_CHECK(t.device_type() == base::DeviceType::kDeviceHIP,
               std::string(name) + " is not on the HIP device");
}

int as_int(size_t n) {
  KUIPER_CHECK(n <= 0x7fffffffu, "size exceeds int32");
  return static_cast<int>(n);
}

// kernels/cpu/add_kernel.cpp:5-19
void add_hip(const tensor::Tensor& in1, const tensor::Tensor& in2, const tensor::Tensor& out,
             void* stream) {
  require_hip(in1, "add input1");
  require_hip(in2, "add input2");
  require_hip(out, "add output");
  KUIPER_CHECK(in1.size() == in2.size() && in1.size() == out.size(), "add size mismatch");
  check_rc(kl_add(in1.ptr<float>(), in2.ptr<float>(), const_cast<float*>(out.ptr<float>()),
                  as_int(in1.size()), stream),
           "kl_add");
}

// kernels/cuda/matmul_kernel.cu:89-109: weight [rows x cols], input [cols].
void matmul_hip(const tensor::Tensor& input, const tensor::Tensor& weight,
                const tensor::Tensor& output, float scale, const HipConfig* config) {
  require_hip(input, "matmul input");
  require_hip(weight, "matmul weight");
  require_hip(output, "matmul output");
  KUIPER_CHECK(weight.dims_size() == 2, "matmul weight must be 2-D");
  const int rows = weight.get_dim(0), cols = weight.get_dim(1);
  KUIPER_CHECK(static_cast<int>(input.size()) == cols, "matmul input size != weight cols");
  KUIPER_CHECK(static_cast<int>(output.size()) == rows, "matmul output size != weight rows");
  check_rc(kl_gemv_f32(input.ptr<float>(), weight.ptr<float>(),
                       const_cast<float*>(output.ptr<float>()), rows, cols, scale,
                       config ? config->stream : nullptr),
           "kl_gemv_f32");
}

// kernels/cuda/matmul_kernel.cu:111-134: int8 weight, fp32 per-group scales.
void matmul_q8_hip(const tensor::Tensor& input, const tensor::Tensor& weight,
                   const tensor::Tensor& output, int32_t group_size, const tensor::Tensor& scale,
                   const HipConfig* config) {
  require_hip(input, "matmul input");
  require_hip(weight, "matmul weight");
  require_hip(scale, "matmul scales");
  require_hip(output, "matmul output");
  KUIPER_CHECK(weight.dims_size() == 2, "matmul weight must be 2-D");
  KUIPER_CHECK(weight.data_type() == base::DataType::kDataTypeInt8, "quant weight must be int8");
  const int rows = weight.get_dim(0), cols = weight.get_dim(1);
  KUIPER_CHECK(static_cast<int>(input.size()) == cols, "matmul input size != weight cols");
  KUIPER_CHECK(static_cast<int>(output.size()) == rows, "matmul output size != weight rows");
  KUIPER_CHECK(group_size > 0 && weight.size() % group_size == 0 &&
                   scale.size() >= weight.size() / group_size,
               "bad group size or scale count");
  check_rc(kl_gemv_q8(input.ptr<float>(), weight.ptr<int8_t>(), scale.ptr<float>(),
                      const_cast<float*>(output.ptr<float>()), rows, cols, group_size,
                      config ? config->stream : nullptr),
           "kl_gemv_q8");
}

// Device staging area for token ids, grown to the largest prompt seen and
// kept for the process (the reference clones the ids into a fresh device
// tensor on every call, emb_kernel.cu:33-35).
struct IdStage {
  int32_t* ptr = nullptr;
  size_t count = 0;
};
IdStage g_ids;

int32_t* stage_ids(size_t n) {
  if (n > g_ids.count) {
    void* p = nullptr;
    const size_t cap = std::max<size_t>(n, 512);
    check_rc(kl_malloc(&p, cap * sizeof(int32_t)), "kl_malloc (token staging)");
    if (g_ids.ptr) kl_free(g_ids.ptr);
    g_ids.ptr = static_cast<int32_t*>(p);
    g_ids.count = cap;
  }
  return g_ids.ptr;
}

// kernels/cuda/emb_kernel.cu:23-48: the token ids arrive in host memory, are
// range-checked on the host (kernels/cpu/emb_kernel.cpp:18-20 CHECKs them) and
// staged to the device.
void embedding_hip(const tensor::Tensor& input, const tensor::Tensor& weight,
                   const tensor::Tensor& output, int32_t vocab_size, void* stream) {
  KUIPER_CHECK(!input.is_empty(), "embedding input is empty");
  require_hip(weight, "embedding weight");
  require_hip(output, "embedding output");
  KUIPER_CHECK(weight.dims_size() == 2 && weight.get_dim(0) == vocab_size,
               "embedding weight must be [vocab x dim]");
  const int dim = weight.get_dim(1);
  const int n = as_int(input.size());
  KUIPER_CHECK(output.size() >= static_cast<size_t>(n) * dim, "embedding output too small");
  const int32_t* ids = nullptr;
  if (input.device_type() == base::DeviceType::kDeviceCPU) {
    for (int i = 0; i < n; ++i) {
      const int32_t t = input.index<int32_t>(i);
      KUIPER_CHECK(t >= 0 && t < vocab_size, "embedding: token id outside [0, vocab)");
    }
    int32_t* staged = stage_ids(n);
    check_rc(kl_memcpy_h2d(staged, input.ptr<int32_t>(), n * sizeof(int32_t), stream),
             "kl_memcpy_h2d");
    ids = staged;
  } else {
    require_hip(input, "embedding input");
    ids = input.ptr<int32_t>();
  }
  check_rc(kl_embedding(ids, n, weight.ptr<float>(), vocab_size, dim,
                        const_cast<float*>(output.ptr<float>()), nullptr, stream),
           "kl_embedding");
  // The host ids may change after return and the staging area is reused by
  // the next call, possibly on another stream.
  if (input.device_type() == base::DeviceType::kDeviceCPU)
    check_rc(kl_stream_sync(stream), "kl_stream_sync");
}

// kernels/cpu/swiglu_kernel.cpp:3-23
void swiglu_hip(const tensor::Tensor& in1, const tensor::Tensor& in2, const tensor::Tensor& out,
                void* stream) {
  require_hip(in1, "swiglu input1");
  require_hip(in2, "swiglu input2");
  require_hip(out, "swiglu output");
  KUIPER_CHECK(in1.size() == in2.size() && in1.size() == out.size(), "swiglu size mismatch");
  check_rc(kl_swiglu(in1.ptr<float>(), in2.ptr<float>(), const_cast<float*>(out.ptr<float>()),
                     as_int(in1.size()), stream),
           "kl_swiglu");
}

// kernels/cuda/mha_kernel.cu:109-127; the score tensor ([head_num x seq_len]
// floats, llama3.cpp:485-487) holds the split partials and needs no
// initialisation.
void mha_hip(int32_t pos, int32_t head_num, int32_t layer_index, int32_t seq_len, int32_t kv_dim,
             int32_t kv_mul, int32_t head_size, const tensor::Tensor& mha_out,
             const tensor::Tensor& query_tensor, const tensor::Tensor& score_tensor,
             const tensor::Tensor& key_cache_tensor, const tensor::Tensor& value_cache_tensor,
             base::DeviceType device_type, HipConfig* config) {
  KUIPER_CHECK(device_type == base::DeviceType::kDeviceHIP, "mha: not a HIP layer");
  require_hip(mha_out, "mha output");
  require_hip(query_tensor, "mha query");
  require_hip(score_tensor, "mha score storage");
  require_hip(key_cache_tensor, "mha key cache");
  require_hip(value_cache_tensor, "mha value cache");
  KUIPER_CHECK(pos >= 0 && pos < seq_len, "mha position out of range");
  const size_t cache_need = static_cast<size_t>(layer_index + 1) * seq_len * kv_dim;
  KUIPER_CHECK(key_cache_tensor.size() >= cache_need && value_cache_tensor.size() >= cache_need,
               "mha caches too small for the layer");
  check_rc(kl_mha(pos, head_num, layer_index, seq_len, kv_dim, kv_mul, head_size,
                  const_cast<float*>(mha_out.ptr<float>()), query_tensor.ptr<float>(),
                  const_cast<void*>(static_cast<const void*>(score_tensor.ptr<float>())),
                  score_tensor.byte_size(), key_cache_tensor.ptr<float>(),
                  value_cache_tensor.ptr<float>(), config ? config->stream : nullptr),
           "kl_mha");
}

// kernels/cpu/rmsnorm_kernel.cpp:4-33
void rmsnorm_hip(const tensor::Tensor& input, const tensor::Tensor& weight,
                 const tensor::Tensor& output, void* stream) {
  require_hip(input, "rmsnorm input");
  require_hip(weight, "rmsnorm weight");
  require_hip(output, "rmsnorm output");
  KUIPER_CHECK(input.size() == weight.size() && input.size() == output.size(),
               "rmsnorm size mismatch");
  check_rc(kl_rmsnorm(input.ptr<float>(), weight.ptr<float>(),
                      const_cast<float*>(output.ptr<float>()), as_int(input.size()),
                      g_traits.rms_eps, stream),
           "kl_rmsnorm");
}

// kernels/cuda/rmsnorm_kernel.cu:138-164: each row of length dim.
void rmsnorm_dim_hip(const tensor::Tensor& input, const tensor::Tensor& weight,
                     const tensor::Tensor& output, int32_t dim, void* stream) {
  require_hip(input, "rmsnorm input");
  require_hip(weight, "rmsnorm weight");
  require_hip(output, "rmsnorm output");
  KUIPER_CHECK(dim > 0 && input.size() % dim == 0 && weight.size() == static_cast<size_t>(dim) &&
                   output.size() == input.size(),
               "rmsnorm_dim size mismatch");
  check_rc(kl_rmsnorm_rows(input.ptr<float>(), weight.ptr<float>(),
                           const_cast<float*>(output.ptr<float>()),
                           as_int(input.size() / dim), dim, g_traits.rms_dim_eps, stream),
           "kl_rmsnorm_rows");
}

// kernels/cpu/rope_kernel.cpp:18-121; pos is read from host memory.
void rope_hip(int32_t dim, int32_t kv_dim, int32_t head_size, const tensor::Tensor& input_q,
              const tensor::Tensor& input_k, const tensor::Tensor& input_pos,
              const tensor::Tensor& sin_cache, const tensor::Tensor& cos_cache, void* stream) {
  require_hip(input_q, "rope query");
  require_hip(input_k, "rope key");
  require_hip(sin_cache, "rope sin cache");
  require_hip(cos_cache, "rope cos cache");
  KUIPER_CHECK(input_pos.device_type() == base::DeviceType::kDeviceCPU,
               "rope position must be in host memory");
  const int32_t pos = input_pos.index<int32_t>(0);
  KUIPER_CHECK(pos >= 0 && static_cast<size_t>(pos + 1) * head_size <= sin_cache.size(),
               "rope position beyond the sin/cos tables");
  KUIPER_CHECK(input_q.size() >= static_cast<size_t>(dim) &&
                   input_k.size() >= static_cast<size_t>(kv_dim),
               "rope tensors too small");
  check_rc(kl_rope(g_traits.rope_style, dim, kv_dim, head_size,
                   const_cast<float*>(input_q.ptr<float>()),
                   const_cast<float*>(input_k.ptr<float>()), pos, sin_cache.ptr<float>(),
                   cos_cache.ptr<float>(), stream),
           "kl_rope");
}

// kernels/cpu/scale_kernel.cpp:3-9: input = input * scale in place.
void scale_hip(float scale, const tensor::Tensor& input, void* stream) {
  require_hip(input, "scale input");
  check_rc(kl_scale(scale, const_cast<float*>(input.ptr<float>()), as_int(input.size()), stream),
           "kl_scale");
}

// kernels/cpu/softmax_kernel.cpp:4-16: softmax of the whole tensor in place.
void softmax_hip(const tensor::Tensor& input, void* stream) {
  require_hip(input, "softmax input");
  check_rc(kl_softmax(const_cast<float*>(input.ptr<float>()), as_int(input.size()), stream),
           "kl_softmax");
}

// kernels/cpu/scale_sum_kernel.cpp:5-22: output += scale[i] * value_i for
// i = 0 .. t, value_i the `size` floats at value + i * stride (the tensor
// `value` is a view of its first row, as mha_kernel.cpp:53-59 builds it).
void scale_sum_hip(const tensor::Tensor& value, const tensor::Tensor& scale,
                   const tensor::Tensor& output, int t, int size, int stride, void* stream) {
  require_hip(value, "scale_sum value");
  require_hip(scale, "scale_sum scale");
  require_hip(output, "scale_sum output");
  KUIPER_CHECK(static_cast<size_t>(size) == value.size() &&
                   static_cast<size_t>(size) == output.size(),
               "scale_sum size mismatch");
  KUIPER_CHECK(t >= 0 && scale.size() > static_cast<size_t>(t), "scale_sum: too few scales");
  check_rc(kl_scale_sum(value.ptr<float>(), scale.ptr<float>(),
                        const_cast<float*>(output.ptr<float>()), t, size, stride, stream),
           "kl_scale_sum");
}
}  // namespace

// kernels/cpu/softmax_kernel.cpp:18-25 (a host function of the interface):
// subtract the maximum, exp, divide by the sum, in place in host memory.  The
// sum adds even and odd elements in two running sums, the order of
// Armadillo's accumulate that the reference's arma::sum uses.
void softmax_inplace_cpu(const float* input_ptr, size_t size) {
  if (!input_ptr || size == 0) return;
  float* x = const_cast<float*>(input_ptr);
  const float mx = *std::max_element(x, x + size);
  for (size_t i = 0; i < size; ++i) x[i] = std::exp(x[i] - mx);
  float even = 0.f, odd = 0.f;
  size_t i = 0;
  for (; i + 1 < size; i += 2) {
    even += x[i];
    odd += x[i + 1];
  }
  if (i < size) even += x[i];
  const float sum = even + odd;
  for (size_t j = 0; j < size; ++j) x[j] = x[j] / sum;
}

void set_kernel_traits(const KernelTraits& traits) { g_traits = traits; }
const KernelTraits& kernel_traits() { return g_traits; }

AddKernel get_add_kernel(base::DeviceType t) {
  return t == base::DeviceType::kDeviceHIP ? add_hip : nullptr;
}
EmbeddingKernel get_emb_kernel(base::DeviceType t) {
  return t == base::DeviceType::kDeviceHIP ? embedding_hip : nullptr;
}
MatmulKernel get_matmul_kernel(base::DeviceType t) {
  return t == base::DeviceType::kDeviceHIP ? matmul_hip : nullptr;
}
MatmulKernelQuant get_matmul_kernel_quant8(base::DeviceType t) {
  return t == base::DeviceType::kDeviceHIP ? matmul_q8_hip : nullptr;
}
MHAKernel get_mha_kernel(base::DeviceType t) {
  return t == base::DeviceType::kDeviceHIP ? mha_hip : nullptr;
}
RMSNormKernel get_rmsnorm_kernel(base::DeviceType t) {
  return t == base::DeviceType::kDeviceHIP ? rmsnorm_hip : nullptr;
}
RMSNormKernelDim get_rmsnorm_dim_kernel(base::DeviceType t) {
  return t == base::DeviceType::kDeviceHIP ? rmsnorm_dim_hip : nullptr;
}
RoPEKernel get_rope_kernel(base::DeviceType t) {
  return t == base::DeviceType::kDeviceHIP ? rope_hip : nullptr;
}
SwigluKernel get_swiglu_kernel(base::DeviceType t, void*) {
  return t == base::DeviceType::kDeviceHIP ? swiglu_hip : nullptr;
}
ScaleKernel get_scale_kernel(base::DeviceType t) {
  return t == base::DeviceType::kDeviceHIP ? scale_hip : nullptr;
}
SoftmaxInplaceKernel get_softmax_kernel(base::DeviceType t) {
  return t == base::DeviceType::kDeviceHIP ? softmax_hip : nullptr;
}
ScaleSumKernel get_scale_sum_kernel(base::DeviceType t) {
  return t == base::DeviceType::kDeviceHIP ? scale_sum_hip : nullptr;
}

void sin_cos_cache_calc_hip(int head_size, int max_seq_len, const tensor::Tensor& sin_cache,
                            const tensor::Tensor& cos_cache) {
  require_hip(sin_cache, "sin cache");
  require_hip(cos_cache, "cos cache");
  KUIPER_CHECK(sin_cache.size() >= static_cast<size_t>(head_size) * max_seq_len &&
                   cos_cache.size() >= static_cast<size_t>(head_size) * max_seq_len,
               "sin/cos tables too small");
  check_rc(kl_sincos_table(head_size, max_seq_len, g_traits.rope_theta,
                           const_cast<float*>(sin_cache.ptr<float>()),
                           const_cast<float*>(cos_cache.ptr<float>())),
           "kl_sincos_table");
}

size_t mha_workspace_bytes(int32_t head_num, int32_t kv_mul, int32_t seq_len, int32_t head_size) {
  size_t bytes = 0;
  check_rc(kl_mha_workspace_size(head_num, kv_mul, seq_len, head_size, &bytes),
           "kl_mha_workspace_size");
  return bytes;
}

}  // namespace kernel
