// Tests of the C++ host API (libkuiper_host.so), after the reference's
// gtest suites test/test_tensor/{test_buffer,test_tensor}.cpp,
// test/test_op/test_cu_{matmul,rmsnorm,add,swiglu,emb}.cpp and
// test/optimized/test_allocator.cpp, plus the model-level driver used by
// tests/test_host_cpp.py.
//
//   test_host unit [prefix]   run the unit tests whose name starts with prefix
//                             ("cpu_" needs no GPU, "hip_" needs one)
//   test_host model <image> <family> <quant> <n_new> <tok0> [tok1 ...]
//       loads the image through model::Model on kDeviceHIP, writes the logits
//       of the first prompt step (layered and fused) to <image>.logits_layered
//       / .logits_fused and prints one JSON line with the greedy tokens of the
//       layered and the fused generate loops.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <memory>
#include <functional>
#include <sstream>
#include <string>
#include <vector>

#include "kuiper/encode.h"
#include "kuiper/kernels.h"
#include "kuiper/layer.h"
#include "kuiper/model.h"
#include "kuiper_hip.h"

namespace {

struct TestCase {
  std::string name;
  std::function<void()> fn;
};
std::vector<TestCase>& registry() {
  static std::vector<TestCase> r;
  return r;
}
struct Register {
  Register(const char* name, std::function<void()> fn) { registry().push_back({name, fn}); }
};
struct Failure {
  std::string what;
};

#define TEST_CASE(name) \
  static void name();   \
  static Register reg_##name(#name, name);

#define EXPECT(cond)                                                                       \
  do {                                                                                     \
    if (!(cond)) throw Failure{std::string(__FILE__ ":") + std::to_string(__LINE__) + ": " + #cond}; \
  } while (0)

#define EXPECT_NEAR(a, b, tol)                                                                \
  do {                                                                                        \
    const double a_ = (a), b_ = (b);                                                          \
    if (!(std::fabs(a_ - b_) <= (tol)))                                                       \
      throw Failure{std::string(__FILE__ ":") + std::to_string(__LINE__) + ": " + #a + "=" + \
                    std::to_string(a_) + " vs " + #b + "=" + std::to_string(b_)};            \
  } while (0)

using base::DataType;
using base::DeviceType;
using tensor::Tensor;

auto cpu_alloc() { return base::CPUDeviceAllocatorFactory::get_instance(); }
auto hip_alloc() { return base::HIPDeviceAllocatorFactory::get_instance(); }

// A deterministic pseudo-random fill in [-1, 1).
void fill(Tensor& t, uint32_t seed) {
  uint32_t s = seed * 2654435761u + 1;
  for (size_t i = 0; i < t.size(); ++i) {
    s = s * 1664525u + 1013904223u;
    t.index<float>(i) = static_cast<float>(s >> 8) / 8388608.f - 1.f;
  }
}

Tensor to_host(const Tensor& t) {
  Tensor c = t.clone();
  c.to_cpu();
  return c;
}

// ----------------------------------------------------------------- cpu_*
TEST_CASE(cpu_buffer_allocate)
void cpu_buffer_allocate() {
  base::Buffer buffer(32, cpu_alloc());
  EXPECT(buffer.ptr() != nullptr);
  EXPECT(!buffer.is_external());
  EXPECT(buffer.device_type() == DeviceType::kDeviceCPU);
}

TEST_CASE(cpu_buffer_use_external)
void cpu_buffer_use_external() {
  std::vector<float> mem(32);
  base::Buffer buffer(32, nullptr, mem.data(), true);
  EXPECT(buffer.is_external());
  EXPECT(buffer.ptr() == mem.data());
}

TEST_CASE(cpu_tensor_init)
void cpu_tensor_init() {
  Tensor t1(DataType::kDataTypeFp32, 32, 32, true, cpu_alloc());
  EXPECT(!t1.is_empty());
  EXPECT(t1.size() == 1024 && t1.byte_size() == 4096);
  EXPECT(t1.strides() == (std::vector<size_t>{32, 1}));
  Tensor t2(DataType::kDataTypeFp32, 32, 32, false, nullptr);
  EXPECT(t2.is_empty());
  std::vector<float> mem(32, 31.f);
  Tensor t3(DataType::kDataTypeFp32, 32, false, nullptr, mem.data());
  EXPECT(!t3.is_empty() && t3.ptr<float>() == mem.data() && *t3.ptr<float>() == 31.f);
}

TEST_CASE(cpu_tensor_assign_clone_reshape)
void cpu_tensor_assign_clone_reshape() {
  Tensor t(DataType::kDataTypeFp32, 32, 32, false, nullptr);
  auto buffer = std::make_shared<base::Buffer>(32 * 32 * sizeof(float), cpu_alloc());
  EXPECT(t.assign(buffer));
  EXPECT(!t.is_empty());
  auto small = std::make_shared<base::Buffer>(16, cpu_alloc());
  EXPECT(!t.assign(small));
  for (int i = 0; i < 1024; ++i) t.index<float>(i) = 1.f;
  Tensor c = t.clone();
  EXPECT(c.ptr<float>() != t.ptr<float>());
  for (int i = 0; i < 1024; ++i) EXPECT(c.index<float>(i) == 1.f);
  c.reshape({64, 16});
  EXPECT(c.get_dim(0) == 64 && c.size() == 1024 && c.index<float>(5) == 1.f);
  c.reshape({4096});
  EXPECT(c.size() == 4096 && c.byte_size() == 4096 * 4);
}

TEST_CASE(cpu_status_codes)
void cpu_status_codes() {
  base::Status ok = base::error::Success();
  EXPECT(bool(ok) && ok.get_err_code() == base::kSuccess);
  base::Status bad = base::error::InvalidArgument("x");
  EXPECT(!bad && bad == base::kInvalidArgument && bad.get_err_msg() == "x");
  EXPECT(base::error::PathNotValid() == base::kPathNotValid);
  EXPECT(base::error::ModelParseError() == base::kModelParseError);
}

TEST_CASE(cpu_kernel_factories)
void cpu_kernel_factories() {
  // Every factory of kernels_interface.h:51-75 has a kDeviceHIP adapter; the
  // reference's CPU and CUDA kernels are not part of this backend.
  const DeviceType H = DeviceType::kDeviceHIP;
  EXPECT(kernel::get_add_kernel(H) && kernel::get_emb_kernel(H) && kernel::get_matmul_kernel(H) &&
         kernel::get_matmul_kernel_quant8(H) && kernel::get_mha_kernel(H) &&
         kernel::get_rmsnorm_kernel(H) && kernel::get_rmsnorm_dim_kernel(H) &&
         kernel::get_rope_kernel(H) && kernel::get_swiglu_kernel(H) && kernel::get_scale_kernel(H) &&
         kernel::get_softmax_kernel(H) && kernel::get_scale_sum_kernel(H));
  for (DeviceType t : {DeviceType::kDeviceCPU, DeviceType::kDeviceCUDA}) {
    EXPECT(kernel::get_matmul_kernel(t) == nullptr && kernel::get_add_kernel(t) == nullptr);
    EXPECT(kernel::get_scale_kernel(t) == nullptr && kernel::get_softmax_kernel(t) == nullptr &&
           kernel::get_scale_sum_kernel(t) == nullptr);
  }
}

TEST_CASE(cpu_softmax_inplace)
void cpu_softmax_inplace() {
  // softmax_kernel.cpp:18-25 on host memory: exp(x - max) / sum.
  std::vector<float> x = {1.f, 2.f, 3.f};
  kernel::softmax_inplace_cpu(x.data(), x.size());
  const double e1 = std::exp(-2.0), e2 = std::exp(-1.0), s = e1 + e2 + 1.0;
  EXPECT_NEAR(x[0], e1 / s, 1e-7);
  EXPECT_NEAR(x[1], e2 / s, 1e-7);
  EXPECT_NEAR(x[2], 1.0 / s, 1e-7);
  std::vector<float> one = {-7.5f};
  kernel::softmax_inplace_cpu(one.data(), 1);
  EXPECT(one[0] == 1.f);  // one element: exp(0) / exp(0)
  std::vector<float> same(9, 3.25f);
  kernel::softmax_inplace_cpu(same.data(), same.size());
  for (float v : same) EXPECT(v == 1.f / 9.f);
}

TEST_CASE(cpu_layer_check_reports_status)
void cpu_layer_check_reports_status() {
  op::MatmulLayer m(DeviceType::kDeviceHIP, 4, 8);
  Tensor in(DataType::kDataTypeFp32, 8, true, cpu_alloc());
  Tensor out(DataType::kDataTypeFp32, 4, true, cpu_alloc());
  // Wrong device: a Status, not an abort.
  base::Status s = m.forward(in, out);
  EXPECT(s == base::kInvalidArgument);
  op::VecAddLayer add(DeviceType::kDeviceHIP);
  EXPECT(add.forward(Tensor(), Tensor(), Tensor()) == base::kInvalidArgument);
}

std::string write_image(const kl_model_spec& spec, const std::string& path, int64_t cut) {
  int64_t bytes = 0;
  if (kl_synth_image_size(&spec, &bytes) != KL_OK) throw Failure{"synth size"};
  std::vector<char> img(bytes);
  if (kl_synth_image(&spec, 7, 0.02f, img.data(), bytes, 1) != KL_OK) throw Failure{"synth"};
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f) throw Failure{"open " + path};
  std::fwrite(img.data(), 1, bytes - cut, f);
  std::fclose(f);
  return path;
}

kl_model_spec tiny_spec(int family) {
  kl_model_spec s{};
  s.family = family;
  s.dim = 64;
  s.q_dim = family == KL_FAMILY_QWEN3 ? 128 : 64;
  s.hidden_dim = 96;
  s.layers = 2;
  s.heads = 4;
  s.kv_heads = 2;
  s.vocab = 100;
  s.seq_len = 32;
  s.tied = 0;
  s.norm_stddev = 0.1f;
  return s;
}

TEST_CASE(cpu_model_errors)
void cpu_model_errors() {
  {
    model::LLama2Model m(base::TokenizerType::kEncodeSpe, "", "/nonexistent/model.bin", false);
    EXPECT(m.init(DeviceType::kDeviceHIP) == base::kPathNotValid);
  }
  {
    model::LLama2Model m(base::TokenizerType::kEncodeSpe, "", "x.bin", false);
    EXPECT(m.init(DeviceType::kDeviceCPU) == base::kInvalidArgument);
  }
  {
    const std::string p = write_image(tiny_spec(KL_FAMILY_LLAMA2), "/tmp/kuiper_host_cut.bin", 64);
    model::LLama2Model m(base::TokenizerType::kEncodeSpe, "", p, false);
    EXPECT(m.init(DeviceType::kDeviceHIP) == base::kModelParseError);
    std::remove(p.c_str());
  }
  {
    kl_model_spec q = tiny_spec(KL_FAMILY_QWEN3);
    const std::string p = write_image(q, "/tmp/kuiper_host_q3.bin", 0);
    model::Qwen3Model m(base::TokenizerType::kEncodeBpe, "", p, true);
    EXPECT(m.init(DeviceType::kDeviceHIP) == base::kInvalidArgument);  // Qwen3 has no int8 layout
    std::remove(p.c_str());
  }
}

// ----------------------------------------------------------------- hip_*
TEST_CASE(hip_buffer_memcpy)
void hip_buffer_memcpy() {
  const int n = 32;
  std::vector<float> src(n);
  for (int i = 0; i < n; ++i) src[i] = float(i);
  base::Buffer host(n * sizeof(float), nullptr, src.data(), true);
  host.set_device_type(DeviceType::kDeviceCPU);
  base::Buffer dev(n * sizeof(float), hip_alloc());
  EXPECT(dev.device_type() == DeviceType::kDeviceHIP);
  dev.copy_from(host);
  base::Buffer dev2(n * sizeof(float), hip_alloc());
  dev2.copy_from(dev);
  base::Buffer back(n * sizeof(float), cpu_alloc());
  back.copy_from(dev2);
  for (int i = 0; i < n; ++i) EXPECT(static_cast<float*>(back.ptr())[i] == float(i));
}

TEST_CASE(hip_tensor_moves)
void hip_tensor_moves() {
  Tensor t(DataType::kDataTypeFp32, 32, 32, true, cpu_alloc());
  for (int i = 0; i < 1024; ++i) t.index<float>(i) = 1.f;
  t.to_hip();
  EXPECT(t.device_type() == DeviceType::kDeviceHIP);
  Tensor c = t.clone();
  EXPECT(c.device_type() == DeviceType::kDeviceHIP && c.ptr<float>() != t.ptr<float>());
  c.to_cpu();
  EXPECT(c.device_type() == DeviceType::kDeviceCPU);
  for (int i = 0; i < 1024; ++i) EXPECT(c.index<float>(i) == 1.f);
}

TEST_CASE(hip_allocator_pool)
void hip_allocator_pool() {
  auto a = hip_alloc();
  void* big = a->allocate(3 << 20);
  EXPECT(big != nullptr);
  a->release(big);
  void* big2 = a->allocate((3 << 20) - 4096);  // within 1 MiB: reused
  EXPECT(big2 == big);
  void* big3 = a->allocate(8 << 20);  // a new block
  EXPECT(big3 != big2);
  void* small = a->allocate(4096);
  a->release(small);
  void* small2 = a->allocate(1000);  // first free small block that fits
  EXPECT(small2 == small);
  a->release(big2);
  a->release(big3);
  a->release(small2);
}

TEST_CASE(hip_matmul_course)
void hip_matmul_course() {
  Tensor in(DataType::kDataTypeFp32, 3, true, cpu_alloc());
  Tensor w(DataType::kDataTypeFp32, 3, 3, true, cpu_alloc());
  in.index<float>(0) = 1.f;
  in.index<float>(1) = 1.f;
  in.index<float>(2) = -1.f;
  for (int i = 1; i <= 9; ++i) w.index<float>(i - 1) = float(i);
  in.to_hip();
  w.to_hip();
  Tensor out(DataType::kDataTypeFp32, 3, true, hip_alloc());
  kernel::get_matmul_kernel(DeviceType::kDeviceHIP)(in, w, out, 1.f, nullptr);
  Tensor h = to_host(out);
  EXPECT(h.index<float>(0) == 0.f && h.index<float>(1) == 3.f && h.index<float>(2) == 6.f);
}

TEST_CASE(hip_matmul_stream_layer)
void hip_matmul_stream_layer() {
  // test_cu_matmul.cpp:matmul_linear_stream5: integers, so the sums are exact.
  kernel::HipConfig config;
  EXPECT(config.create() == KL_OK);
  auto cfg = std::shared_ptr<kernel::HipConfig>(&config, [](kernel::HipConfig*) {});
  for (int rows : {4, 257}) {
    const int cols = rows == 4 ? 4 : 1024;
    std::vector<float> wv(static_cast<size_t>(rows) * cols), xv(cols);
    for (size_t i = 0; i < wv.size(); ++i) wv[i] = float(static_cast<int>(i % 13) - 6);
    for (int i = 0; i < cols; ++i) xv[i] = float(i % 5);
    op::MatmulLayer layer(DeviceType::kDeviceHIP, rows, cols);
    layer.set_weight(0, {rows, cols}, wv.data(), DeviceType::kDeviceCPU);
    layer.set_hip_config(cfg);
    layer.to_hip();
    Tensor x(DataType::kDataTypeFp32, cols, true, cpu_alloc());
    for (int i = 0; i < cols; ++i) x.index<float>(i) = xv[i];
    x.to_hip(config.stream);
    Tensor y(DataType::kDataTypeFp32, rows, true, hip_alloc());
    EXPECT(layer.forward(x, y));
    Tensor h = to_host(y);
    for (int r = 0; r < rows; ++r) {
      double s = 0;
      for (int c = 0; c < cols; ++c) s += double(wv[size_t(r) * cols + c]) * xv[c];
      EXPECT(h.index<float>(r) == float(s));
    }
  }
}

TEST_CASE(hip_matmul_q8_layer)
void hip_matmul_q8_layer() {
  const int rows = 96, cols = 256, gs = 64;
  std::vector<int8_t> blob(static_cast<size_t>(rows) * cols + rows * cols / gs * 4);
  int8_t* q = blob.data();
  float* sc = reinterpret_cast<float*>(blob.data() + rows * cols);
  for (int i = 0; i < rows * cols; ++i) q[i] = static_cast<int8_t>((i * 37) % 255 - 127);
  for (int g = 0; g < rows * cols / gs; ++g) sc[g] = 0.001f * (1 + g % 7);
  op::MatmulLayer layer(DeviceType::kDeviceHIP, rows, cols, true);
  layer.set_group_size(gs);
  layer.set_weight(0, {rows, cols}, blob.data(), DeviceType::kDeviceCPU);
  EXPECT(layer.get_scale_num() == rows * cols / gs);
  layer.to_hip();
  Tensor x(DataType::kDataTypeFp32, cols, true, cpu_alloc());
  fill(x, 3);
  Tensor xh = x.clone();
  x.to_hip();
  Tensor y(DataType::kDataTypeFp32, rows, true, hip_alloc());
  EXPECT(layer.forward(x, y));
  Tensor h = to_host(y);
  for (int r = 0; r < rows; ++r) {
    double s = 0;
    for (int c = 0; c < cols; ++c) {
      const int i = r * cols + c;
      s += double(xh.index<float>(c)) * sc[i / gs] * q[i];
    }
    EXPECT_NEAR(h.index<float>(r), s, 1e-5 * (1 + std::fabs(s)));
  }
}

TEST_CASE(hip_rmsnorm)
void hip_rmsnorm() {
  kernel::set_kernel_traits(kernel::KernelTraits{});
  for (int n : {15, 4096}) {
    Tensor in(DataType::kDataTypeFp32, n, true, cpu_alloc());
    Tensor w(DataType::kDataTypeFp32, n, true, cpu_alloc());
    fill(in, 11);
    fill(w, 12);
    Tensor inh = in.clone(), wh = w.clone();
    in.to_hip();
    w.to_hip();
    Tensor out(DataType::kDataTypeFp32, n, true, hip_alloc());
    kernel::get_rmsnorm_kernel(DeviceType::kDeviceHIP)(in, w, out, nullptr);
    Tensor h = to_host(out);
    double ss = 0;
    for (int i = 0; i < n; ++i) ss += double(inh.index<float>(i)) * inh.index<float>(i);
    const double r = 1.0 / std::sqrt(ss / n + 1e-5);
    for (int i = 0; i < n; ++i)
      EXPECT_NEAR(h.index<float>(i), wh.index<float>(i) * inh.index<float>(i) * r, 1e-5);
  }
}

TEST_CASE(hip_rmsnorm_dim)
void hip_rmsnorm_dim() {
  // test_cu_rmsnorm.cpp:rmsnorm_stream (dim): equal rows give equal outputs.
  const int rows = 32, size = 128;
  Tensor in(DataType::kDataTypeFp32, rows * size, true, cpu_alloc());
  Tensor w(DataType::kDataTypeFp32, size, true, cpu_alloc());
  Tensor row(DataType::kDataTypeFp32, size, true, cpu_alloc());
  fill(row, 5);
  fill(w, 6);
  for (int i = 0; i < rows; ++i)
    for (int j = 0; j < size; ++j) in.index<float>(i * size + j) = row.index<float>(j);
  in.to_hip();
  w.to_hip();
  Tensor out(DataType::kDataTypeFp32, rows * size, true, hip_alloc());
  kernel::get_rmsnorm_dim_kernel(DeviceType::kDeviceHIP)(in, w, out, size, nullptr);
  row.to_hip();
  Tensor golden(DataType::kDataTypeFp32, size, true, hip_alloc());
  // The one-row kernel with the same eps gives the same row.
  kernel::KernelTraits t;
  t.rms_eps = t.rms_dim_eps;
  kernel::set_kernel_traits(t);
  kernel::get_rmsnorm_kernel(DeviceType::kDeviceHIP)(row, w, golden, nullptr);
  kernel::set_kernel_traits(kernel::KernelTraits{});
  Tensor h = to_host(out), g = to_host(golden);
  for (int i = 0; i < rows; ++i)
    for (int j = 0; j < size; ++j) EXPECT_NEAR(h.index<float>(i * size + j), g.index<float>(j), 1e-6);
}

TEST_CASE(hip_add_swiglu)
void hip_add_swiglu() {
  const int n = 32151;  // not a multiple of any vector width
  Tensor a(DataType::kDataTypeFp32, n, true, cpu_alloc());
  Tensor b(DataType::kDataTypeFp32, n, true, cpu_alloc());
  for (int i = 0; i < n; ++i) {
    a.index<float>(i) = 2.f;
    b.index<float>(i) = 3.f;
  }
  Tensor ah = a.clone();
  fill(ah, 21);
  Tensor bh = b.clone();
  fill(bh, 22);
  a.to_hip();
  b.to_hip();
  Tensor out(DataType::kDataTypeFp32, n, true, hip_alloc());
  kernel::get_add_kernel(DeviceType::kDeviceHIP)(a, b, out, nullptr);
  Tensor h = to_host(out);
  for (int i = 0; i < n; ++i) EXPECT(h.index<float>(i) == 5.f);
  Tensor a2 = ah.clone(), b2 = bh.clone();
  a2.to_hip();
  b2.to_hip();
  op::SwiGLULayer sw(DeviceType::kDeviceHIP, n);
  EXPECT(sw.forward(a2, b2, a2));  // in place, as llama3.cpp:707
  Tensor s = to_host(a2);
  for (int i = 0; i < n; ++i) {
    const double x = ah.index<float>(i);
    EXPECT_NEAR(s.index<float>(i), x / (1 + std::exp(-x)) * bh.index<float>(i), 1e-6);
  }
}

TEST_CASE(hip_mha_from_building_blocks)
void hip_mha_from_building_blocks() {
  // The reference's CPU MHA (kernels/cpu/mha_kernel.cpp:5-61) written the
  // reference's way, from factory kernels on kDeviceHIP tensors: per head, a
  // 1-row matmul per position (score = q . K_t / sqrt(hd)), the in-place
  // softmax, a zeroed output and the scale-sum over V rows.  It must agree
  // with the fused MHA kernel on the same caches.
  const int head_num = 8, kv_mul = 4, head_size = 64, seq_len = 96, layer = 1, pos = 70;
  const int kv_dim = head_num / kv_mul * head_size;
  auto alloc = hip_alloc();
  Tensor q(DataType::kDataTypeFp32, head_num * head_size, true, cpu_alloc());
  Tensor kc(DataType::kDataTypeFp32, 2 * seq_len * kv_dim, true, cpu_alloc());
  Tensor vc(DataType::kDataTypeFp32, 2 * seq_len * kv_dim, true, cpu_alloc());
  fill(q, 31);
  fill(kc, 32);
  fill(vc, 33);
  q.to_hip();
  kc.to_hip();
  vc.to_hip();
  Tensor score(DataType::kDataTypeFp32, head_num * seq_len, true, alloc);
  Tensor out(DataType::kDataTypeFp32, head_num * head_size, true, alloc);
  const DeviceType H = DeviceType::kDeviceHIP;
  auto view = [&](const float* p, std::vector<int32_t> dims) {
    Tensor t(DataType::kDataTypeFp32, dims, false, nullptr, const_cast<float*>(p));
    t.set_device_type(H);
    return t;
  };
  const float scale = 1.f / std::sqrt(static_cast<float>(head_size));
  const size_t layer_off = static_cast<size_t>(layer) * seq_len * kv_dim;
  for (int h = 0; h < head_num; ++h) {
    float* sh = score.ptr<float>() + h * seq_len;
    Tensor qh = view(q.ptr<float>() + h * head_size, {head_size});
    for (int t = 0; t <= pos; ++t) {
      const float* kt = kc.ptr<float>() + layer_off + t * kv_dim + (h / kv_mul) * head_size;
      kernel::get_matmul_kernel(H)(qh, view(kt, {1, head_size}), view(sh + t, {1}), scale, nullptr);
    }
    Tensor sc = view(sh, {pos + 1});
    kernel::get_softmax_kernel(H)(sc, nullptr);
    float* oh = out.ptr<float>() + h * head_size;
    alloc->memset_zero(oh, sizeof(float) * head_size, nullptr, false);
    const float* vh = vc.ptr<float>() + layer_off + (h / kv_mul) * head_size;
    kernel::get_scale_sum_kernel(H)(view(vh, {head_size}), sc, view(oh, {head_size}), pos,
                                    head_size, kv_dim, nullptr);
  }
  Tensor ws(DataType::kDataTypeFp32,
            static_cast<int32_t>(kernel::mha_workspace_bytes(head_num, kv_mul, seq_len, head_size) / 4) + 1,
            true, alloc);
  alloc->memset_zero(ws.ptr<float>(), ws.byte_size(), nullptr, true);
  Tensor fused(DataType::kDataTypeFp32, head_num * head_size, true, alloc);
  kernel::get_mha_kernel(H)(pos, head_num, layer, seq_len, kv_dim, kv_mul, head_size, fused, q, ws, kc,
                            vc, H, nullptr);
  Tensor a = to_host(out), b = to_host(fused);
  for (int i = 0; i < head_num * head_size; ++i) EXPECT_NEAR(a.index<float>(i), b.index<float>(i), 2e-6);
  // The scale kernel: x * scale in place, one rounding.
  Tensor x(DataType::kDataTypeFp32, 1000, true, cpu_alloc());
  fill(x, 34);
  Tensor xh = x.clone();
  x.to_hip();
  kernel::get_scale_kernel(H)(0.375f, x, nullptr);
  Tensor y = to_host(x);
  for (int i = 0; i < 1000; ++i) EXPECT(y.index<float>(i) == xh.index<float>(i) * 0.375f);
}

TEST_CASE(hip_embedding)
void hip_embedding() {
  // test_cu_emb.cpp:emb1_nostream: row 1 of a [vocab x 512] table of i.
  const int vocab = 4, dim = 512;
  op::EmbeddingLayer layer(DeviceType::kDeviceHIP, dim, 16, vocab);
  std::vector<float> table(vocab * dim);
  for (int i = 0; i < vocab * dim; ++i) table[i] = float(i);
  layer.set_weight(0, {vocab, dim}, table.data(), DeviceType::kDeviceCPU);
  layer.to_hip();
  Tensor ids(DataType::kDataTypeInt32, 2, true, cpu_alloc());
  ids.index<int32_t>(0) = 1;
  ids.index<int32_t>(1) = 3;
  Tensor num(DataType::kDataTypeInt32, 2);
  Tensor out(DataType::kDataTypeFp32, 2, dim, true, hip_alloc());
  EXPECT(layer.forward(ids, num, out));
  Tensor h = to_host(out);
  for (int i = 0; i < dim; ++i) {
    EXPECT(h.index<float>(i) == float(512 + i));
    EXPECT(h.index<float>(dim + i) == float(3 * 512 + i));
  }
  // Too few ids for the count: a Status.
  Tensor num3(DataType::kDataTypeInt32, 3);
  EXPECT(layer.forward(ids, num3, out) == base::kInvalidArgument);
}

TEST_CASE(hip_argmax_sampler)
void hip_argmax_sampler() {
  const int n = 128256;
  Tensor x(DataType::kDataTypeFp32, n, true, cpu_alloc());
  fill(x, 9);
  x.index<float>(77777) = 5.f;
  x.index<float>(99999) = 5.f;  // a tie: the first index wins
  Tensor xd = x.clone();
  xd.to_hip();
  sampler::ArgmaxSampler s(DeviceType::kDeviceHIP);
  EXPECT(s.sample(xd.ptr<float>(), n, nullptr) == 77777);
  sampler::ArgmaxSampler c(DeviceType::kDeviceCPU);
  EXPECT(c.sample(x.ptr<float>(), n, nullptr) == 77777);
}

int run_units(const std::string& prefix) {
  int failed = 0, ran = 0;
  for (auto& t : registry()) {
    if (t.name.compare(0, prefix.size(), prefix) != 0) continue;
    ++ran;
    try {
      t.fn();
      std::printf("[ OK ] %s\n", t.name.c_str());
    } catch (const Failure& f) {
      ++failed;
      std::printf("[FAIL] %s: %s\n", t.name.c_str(), f.what.c_str());
    }
    std::fflush(stdout);
  }
  std::printf("%d tests, %d failed\n", ran, failed);
  return failed == 0 && ran > 0 ? 0 : 1;
}

void write_floats(const std::string& path, const Tensor& t) {
  Tensor h = to_host(t);
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f) base::fatal(__FILE__, __LINE__, "cannot write " + path);
  std::fwrite(h.ptr<float>(), sizeof(float), h.size(), f);
  std::fclose(f);
}

std::string join(const std::vector<int32_t>& v) {
  std::string s = "[";
  for (size_t i = 0; i < v.size(); ++i) s += (i ? "," : "") + std::to_string(v[i]);
  return s + "]";
}

// A reference-style subclass (include/model/llama3.h:33-53 overrides
// predict): counts its predict() calls and forwards them.  Model::generate
// must reach it through the virtual interface.
template <class Base>
class CountingModel : public Base {
 public:
  using Base::Base;
  base::Status predict(const tensor::Tensor& input, const tensor::Tensor& pos_tensor,
                       bool is_prompt, int& next) const override {
    ++calls;
    return Base::predict(input, pos_tensor, is_prompt, next);
  }
  mutable int calls = 0;
};

template <class M>
std::pair<std::vector<int32_t>, int> counted_generate(M* m, const std::vector<int32_t>& prompt,
                                                      int n_new) {
  STATUS_CHECK(m->init(DeviceType::kDeviceHIP));
  std::vector<int32_t> out;
  STATUS_CHECK(static_cast<const model::Model*>(m)->generate(prompt, n_new, out));
  return {out, m->calls};
}

int run_model(int argc, char** argv) {
  if (argc < 7) {
    std::fprintf(stderr, "usage: model <image> <family> <quant> <n_new> <tok0> [tok...]\n");
    return 2;
  }
  const std::string path = argv[2];
  const auto family = static_cast<model::ModelFamily>(std::atoi(argv[3]));
  const bool quant = std::atoi(argv[4]) != 0;
  const int n_new = std::atoi(argv[5]);
  std::vector<int32_t> prompt;
  for (int i = 6; i < argc; ++i) prompt.push_back(std::atoi(argv[i]));

  std::unique_ptr<model::Model> m;
  if (family == model::ModelFamily::kQwen2)
    m = std::make_unique<model::Qwen2Model>(base::TokenizerType::kEncodeBpe, "", path, quant);
  else if (family == model::ModelFamily::kQwen3)
    m = std::make_unique<model::Qwen3Model>(base::TokenizerType::kEncodeBpe, "", path, quant);
  else
    m = std::make_unique<model::LLama2Model>(base::TokenizerType::kEncodeSpe, "", path, quant,
                                             family);
  STATUS_CHECK(m->init(DeviceType::kDeviceHIP));

  // The first prompt step, as demo/main.cpp drives it.
  tensor::Tensor pos = m->get_buffer(model::ModelBufferType::kInputPos);
  pos.index<int32_t>(0) = 0;
  int next = -1;
  {
    const op::EmbeddingOutput emb = m->embedding(prompt);
    STATUS_CHECK(m->predict(m->fill_input(pos, emb, true), pos, true, next));
    write_floats(path + ".logits_layered", m->get_buffer(model::ModelBufferType::kForwardOutput));
  }
  std::vector<int32_t> layered, fused;
  STATUS_CHECK(m->generate(prompt, n_new, layered));

  STATUS_CHECK(m->set_fused(true));
  pos.index<int32_t>(0) = 0;
  {
    const op::EmbeddingOutput emb = m->embedding(prompt);
    STATUS_CHECK(m->predict(m->fill_input(pos, emb, true), pos, true, next));
    write_floats(path + ".logits_fused", m->get_buffer(model::ModelBufferType::kForwardOutput));
  }
  STATUS_CHECK(m->generate(prompt, n_new, fused));
  // The fused predict() path driven token by token (not kl_engine_generate).
  std::vector<int32_t> fused_steps;
  {
    const op::EmbeddingOutput pe = m->embedding(prompt);
    const int P = static_cast<int>(prompt.size());
    for (int p = 0; p < P - 1; ++p) {
      pos.index<int32_t>(0) = p;
      STATUS_CHECK(m->predict(m->fill_input(pos, pe, true), pos, true, next));
    }
    int32_t tok = prompt[P - 1];
    for (int i = 0; i < n_new; ++i) {
      pos.index<int32_t>(0) = P - 1 + i;
      const op::EmbeddingOutput e = m->embedding({tok});
      STATUS_CHECK(m->predict(m->fill_input(pos, e, false), pos, false, next));
      fused_steps.push_back(next);
      tok = next;
    }
  }
  // The same loop through a subclass that overrides predict().
  std::pair<std::vector<int32_t>, int> sub;
  if (family == model::ModelFamily::kQwen2) {
    CountingModel<model::Qwen2Model> cm(base::TokenizerType::kEncodeBpe, "", path, quant);
    sub = counted_generate(&cm, prompt, n_new);
  } else if (family == model::ModelFamily::kQwen3) {
    CountingModel<model::Qwen3Model> cm(base::TokenizerType::kEncodeBpe, "", path, quant);
    sub = counted_generate(&cm, prompt, n_new);
  } else {
    CountingModel<model::LLama2Model> cm(base::TokenizerType::kEncodeSpe, "", path, quant, family);
    sub = counted_generate(&cm, prompt, n_new);
  }
  const auto& c = m->config();
  std::printf("{\"dims\": [%d, %d, %d, %d, %d, %d, %d, %d], \"layered\": %s, \"fused\": %s, "
              "\"fused_steps\": %s, \"subclass\": %s, \"subclass_predict_calls\": %d, "
              "\"pooled_bytes\": %zu}\n",
              c.dim_, c.q_dim_, c.kv_dim_, c.hidden_dim_, c.layer_num_, c.head_num_,
              c.kv_head_num_, c.vocab_size_, join(layered).c_str(), join(fused).c_str(),
              join(fused_steps).c_str(), join(sub.first).c_str(), sub.second,
              base::HIPDeviceAllocatorFactory::get_instance()->pooled_bytes());
  return 0;
}

}  // namespace

// tok <spe|bpe|qwen> <tokenizer file> <cases file>: the tokenizer layers
// (op::SpeEncodeLayer / BpeEncodeLayer / QwenEncodeLayer) on the cases, one
// per line as hex-encoded UTF-8 ("-" = empty).  Prints a "meta" line, then
// per case "ids <ids...>", "dec <hex of decode(ids)>" and "end <0|1>"; a line
// "#<ids...>" is decoded only and prints "only <hex of decode(ids)>".
static std::string hex_to_bytes(const std::string& h) {
  std::string out;
  if (h == "-") return out;
  for (size_t i = 0; i + 1 < h.size(); i += 2) out += static_cast<char>(std::stoi(h.substr(i, 2), nullptr, 16));
  return out;
}

static int run_tok(int argc, char** argv) {
  if (argc < 5) {
    std::fprintf(stderr, "usage: test_host tok <spe|bpe|qwen> <tokenizer> <cases>\n");
    return 2;
  }
  const std::string kind = argv[2];
  std::unique_ptr<op::EncodeLayerBase> layer;
  if (kind == "spe") layer = std::make_unique<op::SpeEncodeLayer>(argv[3], true, false);
  else if (kind == "bpe") layer = std::make_unique<op::BpeEncodeLayer>(argv[3], true, false);
  else layer = std::make_unique<op::QwenEncodeLayer>(argv[3], false, false);
  const base::Status st = layer->init();
  std::printf("meta init %d vocab %d\n", static_cast<int>(st), layer->vocab_size());
  if (!st) {
    std::printf("error %s\n", st.get_err_msg().c_str());
    return 1;
  }
  std::ifstream f(argv[4]);
  std::string line;
  while (std::getline(f, line)) {
    if (!line.empty() && line[0] == '#') {  // "#id id ...": decode only
      std::vector<int32_t> ids;
      std::istringstream in(line.substr(1));
      for (int32_t id; in >> id;) ids.push_back(id);
      std::printf("only ");
      for (unsigned char ch : layer->decode(ids)) std::printf("%02x", ch);
      std::printf("\n");
      continue;
    }
    const std::vector<int32_t> ids = layer->encode(hex_to_bytes(line));
    std::printf("ids");
    for (int32_t id : ids) std::printf(" %d", id);
    std::printf("\ndec ");
    for (unsigned char ch : layer->decode(ids)) std::printf("%02x", ch);
    std::printf("\nend %d\n", ids.empty() ? 0 : static_cast<int>(layer->is_sentence_ending(ids.back())));
  }
  return 0;
}

int main(int argc, char** argv) {
  const std::string mode = argc > 1 ? argv[1] : "unit";
  if (mode == "unit") return run_units(argc > 2 ? argv[2] : "");
  if (mode == "model") return run_model(argc, argv);
  if (mode == "tok") return run_tok(argc, argv);
  std::fprintf(stderr, "unknown mode %s\n", mode.c_str());
  return 2;
}
