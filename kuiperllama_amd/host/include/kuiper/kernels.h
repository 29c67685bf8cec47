// Kernel dispatch of the host API: the reference's function-pointer typedefs
// (source/op/kernels/kernels_interface.h:6-49) and get_*_kernel(DeviceType)
// factories (kernels_interface.h:51-75, kernels_interfaces.cpp:21-141).  For
// kDeviceHIP each factory returns an adapter that unpacks the Tensors into a
// call of the C ABI (include/kuiper_hip.h); the reference's own CPU/CUDA
// kernels are not part of this backend, so other device types return nullptr.
#pragma once
#include "kuiper/hip_config.h"
#include "kuiper/tensor.h"

namespace kernel {

typedef void (*AddKernel)(const tensor::Tensor& input1, const tensor::Tensor& input2,
                          const tensor::Tensor& output, void* stream);
typedef void (*MatmulKernel)(const tensor::Tensor& input, const tensor::Tensor& weight,
                             const tensor::Tensor& output, float scale, const HipConfig* config);
typedef void (*MatmulKernelQuant)(const tensor::Tensor& input, const tensor::Tensor& weight,
                                  const tensor::Tensor& output, int32_t group_size,
                                  const tensor::Tensor& scale, const HipConfig* config);
typedef void (*EmbeddingKernel)(const tensor::Tensor& input, const tensor::Tensor& weight,
                                const tensor::Tensor& output, int32_t vocab_size, void* stream);
typedef void (*SwigluKernel)(const tensor::Tensor& input1, const tensor::Tensor& input2,
                             const tensor::Tensor& output, void* stream);
typedef void (*MHAKernel)(int32_t pos, int32_t head_num, int32_t layer_index, int32_t seq_len,
                          int32_t kv_dim, int32_t kv_mul, int32_t head_size,
                          const tensor::Tensor& mha_out, const tensor::Tensor& query_tensor,
                          const tensor::Tensor& score_tensor,
                          const tensor::Tensor& key_cache_tensor,
                          const tensor::Tensor& value_cache_tensor, base::DeviceType device_type,
                          HipConfig*);
typedef void (*RMSNormKernel)(const tensor::Tensor& input, const tensor::Tensor& weight,
                              const tensor::Tensor& output, void* stream);
typedef void (*RMSNormKernelDim)(const tensor::Tensor& input, const tensor::Tensor& weight,
                                 const tensor::Tensor& output, int32_t dim, void* stream);
typedef void (*RoPEKernel)(int32_t dim, int32_t kv_dim, int32_t head_size,
                           const tensor::Tensor& input_q, const tensor::Tensor& input_k,
                           const tensor::Tensor& input_pos, const tensor::Tensor& sin_cache,
                           const tensor::Tensor& cos_cache, void* stream);
// The CPU MHA's building blocks (kernels_interface.h:41-49): in-place scale,
// in-place softmax of a whole tensor, and output += sum_i scale[i] * value_i
// over rows i = 0 .. t of `size` floats at a stride.
typedef void (*ScaleKernel)(float scale, const tensor::Tensor& input, void* stream);
typedef void (*SoftmaxInplaceKernel)(const tensor::Tensor& input, void* stream);
typedef void (*ScaleSumKernel)(const tensor::Tensor& value, const tensor::Tensor& scale,
                               const tensor::Tensor& output, int t, int size, int stride,
                               void* stream);

// Softmax in place over `size` floats in host memory (kernels_interface.h:49).
void softmax_inplace_cpu(const float* input_ptr, size_t size);

// What the reference fixes with -DLLAMA3_SUPPORT / -DQWEN2_SUPPORT /
// -DQWEN3_SUPPORT (RoPE pairing and theta, RMSNorm eps; see
// kernels/cpu/rope_kernel.cpp:3-122, kernels/cpu/rmsnorm_kernel.cpp:24-28)
// as process-wide runtime values, set by a model's init().
struct KernelTraits {
  int rope_style = 0;      // KL_ROPE_INTERLEAVED / KL_ROPE_HALF
  float rope_theta = 1e4f;
  float rms_eps = 1e-5f;
  float rms_dim_eps = 1e-6f;  // per-row (q/k) RMSNorm, kernels/cuda/rmsnorm_kernel.cu:148
};
void set_kernel_traits(const KernelTraits& traits);
const KernelTraits& kernel_traits();

AddKernel get_add_kernel(base::DeviceType device_type);
EmbeddingKernel get_emb_kernel(base::DeviceType device_type);
MatmulKernel get_matmul_kernel(base::DeviceType device_type);
MatmulKernelQuant get_matmul_kernel_quant8(base::DeviceType device_type);
MHAKernel get_mha_kernel(base::DeviceType device_type);
RMSNormKernel get_rmsnorm_kernel(base::DeviceType device_type);
RMSNormKernelDim get_rmsnorm_dim_kernel(base::DeviceType device_type);
RoPEKernel get_rope_kernel(base::DeviceType device_type);
SwigluKernel get_swiglu_kernel(base::DeviceType device_type, void* stream = nullptr);
ScaleKernel get_scale_kernel(base::DeviceType device_type);
SoftmaxInplaceKernel get_softmax_kernel(base::DeviceType device_type);
ScaleSumKernel get_scale_sum_kernel(base::DeviceType device_type);

// sin_cos_cache_calc (kernels/cpu/rope_kernel.cpp:4-16): fills the device
// tables [seq_len x head_size] with the reference's float formula.
void sin_cos_cache_calc_hip(int head_size, int max_seq_len, const tensor::Tensor& sin_cache,
                            const tensor::Tensor& cos_cache);

// Bytes the MHA kernel needs in its score tensor (the split-K workspace);
// the tensor must be zeroed once before its first use.
size_t mha_workspace_bytes(int32_t head_num, int32_t kv_mul, int32_t seq_len, int32_t head_size);

}  // namespace kernel
