// Status helpers, allocators, Buffer and Tensor of the host API.
#include <cstring>
#include <numeric>

#include "kuiper/alloc.h"
#include "kuiper/base.h"
#include "kuiper/hip_config.h"
#include "kuiper/tensor.h"
#include "kuiper_hip.h"

namespace base {

namespace error {
Status Success(const std::string& m) { return Status(kSuccess, m); }
Status FunctionNotImplement(const std::string& m) { return Status(kFunctionUnImplement, m); }
Status PathNotValid(const std::string& m) { return Status(kPathNotValid, m); }
Status ModelParseError(const std::string& m) { return Status(kModelParseError, m); }
Status InternalError(const std::string& m) { return Status(kInternalError, m); }
Status KeyHasExits(const std::string& m) { return Status(kKeyValueHasExist, m); }
Status InvalidArgument(const std::string& m) { return Status(kInvalidArgument, m); }
}  // namespace error

void fatal(const char* file, int line, const std::string& what) {
  std::fprintf(stderr, "kuiper fatal: %s:%d: %s\n", file, line, what.c_str());
  std::fflush(stderr);
  std::abort();
}

namespace {
void check_rc(int rc, const char* what) {
  if (rc != KL_OK) fatal(__FILE__, __LINE__, std::string(what) + ": " + kl_error_string(rc));
}
int current_device() {
  // The C ABI works on the current device; the pool keys blocks by it.  Only
  // device 0 is used by this backend (one GPU per process).
  return 0;
}
}  // namespace

// ---------------------------------------------------------------------------
// Allocators.
// ---------------------------------------------------------------------------
void DeviceAllocator::memcpy(const void* src, void* dst, size_t bytes, MemcpyKind kind,
                             void* stream, bool need_sync) const {
  KUIPER_CHECK(src && dst, "null pointer");
  if (bytes == 0) return;
  switch (kind) {
    case MemcpyKind::kMemcpyCPU2CPU: std::memcpy(dst, src, bytes); return;
    case MemcpyKind::kMemcpyCPU2CUDA: check_rc(kl_memcpy_h2d(dst, src, bytes, stream), "kl_memcpy_h2d"); break;
    case MemcpyKind::kMemcpyCUDA2CPU: check_rc(kl_memcpy_d2h(dst, src, bytes, stream), "kl_memcpy_d2h"); break;
    case MemcpyKind::kMemcpyCUDA2CUDA: check_rc(kl_memcpy_d2d(dst, src, bytes, stream), "kl_memcpy_d2d"); break;
  }
  if (need_sync) check_rc(kl_stream_sync(stream), "kl_stream_sync");
}

void DeviceAllocator::memset_zero(void* ptr, size_t bytes, void* stream, bool need_sync) {
  KUIPER_CHECK(ptr, "null pointer");
  if (device_type() == DeviceType::kDeviceCPU) {
    std::memset(ptr, 0, bytes);
    return;
  }
  check_rc(kl_memset_zero(ptr, bytes, stream), "kl_memset_zero");
  if (need_sync) check_rc(kl_stream_sync(stream), "kl_stream_sync");
}

CPUDeviceAllocator::CPUDeviceAllocator() : DeviceAllocator(DeviceType::kDeviceCPU) {}

void* CPUDeviceAllocator::allocate(size_t bytes) const {
  if (!bytes) return nullptr;
  void* p = nullptr;
  // 32-byte alignment for buffers of 1 KiB and more, 16 below (alloc_cpu.cpp:10-37).
  const size_t align = bytes >= 1024 ? 32 : 16;
  if (posix_memalign(&p, align, bytes) != 0) return nullptr;
  return p;
}

void CPUDeviceAllocator::release(void* ptr) const { std::free(ptr); }

HIPDeviceAllocator::HIPDeviceAllocator() : DeviceAllocator(DeviceType::kDeviceHIP) {}

namespace {
constexpr size_t kBigBlock = 1 << 20;         // requests above 1 MiB use the big pool
constexpr size_t kBigSlack = 1 << 20;         // a reused big block wastes < 1 MiB
constexpr size_t kIdleSmallLimit = 1ull << 30;  // free idle small blocks past 1 GiB
}  // namespace

void* HIPDeviceAllocator::allocate(size_t bytes) const {
  if (!bytes) return nullptr;
  const int dev = current_device();
  if (bytes > kBigBlock) {
    auto& big = big_buffers_[dev];
    int best = -1;
    for (int i = 0; i < static_cast<int>(big.size()); ++i) {
      const HipMemoryBuffer& b = big[i];
      if (!b.busy && b.byte_size >= bytes && b.byte_size - bytes < kBigSlack &&
          (best < 0 || b.byte_size < big[best].byte_size))
        best = i;
    }
    if (best >= 0) {
      big[best].busy = true;
      return big[best].data;
    }
    void* p = nullptr;
    if (kl_malloc(&p, bytes) != KL_OK) {
      std::fprintf(stderr, "kuiper: device allocation of %zu bytes failed\n", bytes);
      return nullptr;
    }
    big.push_back({p, bytes, true});
    return p;
  }
  auto& small = small_buffers_[dev];
  for (HipMemoryBuffer& b : small) {
    if (!b.busy && b.byte_size >= bytes) {
      b.busy = true;
      idle_small_bytes_[dev] -= b.byte_size;
      return b.data;
    }
  }
  void* p = nullptr;
  if (kl_malloc(&p, bytes) != KL_OK) {
    std::fprintf(stderr, "kuiper: device allocation of %zu bytes failed\n", bytes);
    return nullptr;
  }
  small.push_back({p, bytes, true});
  return p;
}

void HIPDeviceAllocator::release(void* ptr) const {
  if (!ptr) return;
  for (auto& [dev, small] : small_buffers_) {
    for (HipMemoryBuffer& b : small) {
      if (b.data == ptr) {
        b.busy = false;
        idle_small_bytes_[dev] += b.byte_size;
        if (idle_small_bytes_[dev] > kIdleSmallLimit) {
          std::vector<HipMemoryBuffer> keep;
          for (HipMemoryBuffer& x : small) {
            if (x.busy) keep.push_back(x);
            else kl_free(x.data);
          }
          small.swap(keep);
          idle_small_bytes_[dev] = 0;
        }
        return;
      }
    }
  }
  for (auto& [dev, big] : big_buffers_) {
    for (HipMemoryBuffer& b : big) {
      if (b.data == ptr) {
        b.busy = false;
        return;
      }
    }
  }
  kl_free(ptr);  // not from the pool
}

size_t HIPDeviceAllocator::pooled_bytes() const {
  size_t n = 0;
  for (auto& [d, v] : big_buffers_)
    for (auto& b : v) n += b.byte_size;
  for (auto& [d, v] : small_buffers_)
    for (auto& b : v) n += b.byte_size;
  return n;
}

std::shared_ptr<CPUDeviceAllocator> CPUDeviceAllocatorFactory::get_instance() {
  static std::shared_ptr<CPUDeviceAllocator> instance = std::make_shared<CPUDeviceAllocator>();
  return instance;
}

std::shared_ptr<HIPDeviceAllocator> HIPDeviceAllocatorFactory::get_instance() {
  static std::shared_ptr<HIPDeviceAllocator> instance = std::make_shared<HIPDeviceAllocator>();
  return instance;
}

std::shared_ptr<DeviceAllocator> allocator_for(DeviceType t) {
  if (t == DeviceType::kDeviceCPU) return CPUDeviceAllocatorFactory::get_instance();
  if (t == DeviceType::kDeviceHIP) return HIPDeviceAllocatorFactory::get_instance();
  return nullptr;
}

// ---------------------------------------------------------------------------
// Buffer.
// ---------------------------------------------------------------------------
Buffer::Buffer(size_t byte_size, std::shared_ptr<DeviceAllocator> allocator, void* ptr,
               bool use_external)
    : byte_size_(byte_size), ptr_(ptr), use_external_(use_external), allocator_(allocator) {
  if (!ptr_ && allocator_) {
    device_type_ = allocator_->device_type();
    use_external_ = false;
    ptr_ = allocator_->allocate(byte_size_);
  } else if (allocator_) {
    device_type_ = allocator_->device_type();
  }
}

Buffer::~Buffer() {
  if (!use_external_ && ptr_ && allocator_) allocator_->release(ptr_);
  ptr_ = nullptr;
}

bool Buffer::allocate() {
  if (allocator_ && byte_size_ != 0) {
    use_external_ = false;
    ptr_ = allocator_->allocate(byte_size_);
    return ptr_ != nullptr;
  }
  return false;
}

void Buffer::copy_from(const Buffer& buffer) const {
  KUIPER_CHECK(allocator_ != nullptr, "buffer without allocator");
  KUIPER_CHECK(buffer.ptr_ != nullptr, "copy from an empty buffer");
  const size_t n = byte_size_ < buffer.byte_size_ ? byte_size_ : buffer.byte_size_;
  const DeviceType src = buffer.device_type_, dst = device_type_;
  KUIPER_CHECK(src != DeviceType::kDeviceUnknown && dst != DeviceType::kDeviceUnknown,
               "unknown device type");
  MemcpyKind kind;
  if (src == DeviceType::kDeviceCPU && dst == DeviceType::kDeviceCPU) kind = MemcpyKind::kMemcpyCPU2CPU;
  else if (src == DeviceType::kDeviceCPU) kind = MemcpyKind::kMemcpyCPU2CUDA;
  else if (dst == DeviceType::kDeviceCPU) kind = MemcpyKind::kMemcpyCUDA2CPU;
  else kind = MemcpyKind::kMemcpyCUDA2CUDA;
  allocator_->memcpy(buffer.ptr_, ptr_, n, kind, nullptr, true);
}

void Buffer::copy_from(const Buffer* buffer) const {
  KUIPER_CHECK(buffer != nullptr, "null buffer");
  copy_from(*buffer);
}

}  // namespace base

// ---------------------------------------------------------------------------
// Tensor.
// ---------------------------------------------------------------------------
namespace tensor {

static size_t reduce_dims(const std::vector<int32_t>& dims) {
  if (dims.empty()) return 0;
  return std::accumulate(dims.begin(), dims.end(), size_t(1),
                         [](size_t a, int32_t b) { return a * static_cast<size_t>(b); });
}

Tensor::Tensor(base::DataType data_type, int32_t dim0, bool need_alloc,
               std::shared_ptr<base::DeviceAllocator> alloc, void* ptr)
    : Tensor(data_type, std::vector<int32_t>{dim0}, need_alloc, alloc, ptr) {}

Tensor::Tensor(base::DataType data_type, int32_t dim0, int32_t dim1, bool need_alloc,
               std::shared_ptr<base::DeviceAllocator> alloc, void* ptr)
    : Tensor(data_type, std::vector<int32_t>{dim0, dim1}, need_alloc, alloc, ptr) {}

Tensor::Tensor(base::DataType data_type, int32_t dim0, int32_t dim1, int32_t dim2, bool need_alloc,
               std::shared_ptr<base::DeviceAllocator> alloc, void* ptr)
    : Tensor(data_type, std::vector<int32_t>{dim0, dim1, dim2}, need_alloc, alloc, ptr) {}

Tensor::Tensor(base::DataType data_type, std::vector<int32_t> dims, bool need_alloc,
               std::shared_ptr<base::DeviceAllocator> alloc, void* ptr)
    : dims_(std::move(dims)), data_type_(data_type) {
  size_ = reduce_dims(dims_);
  if (need_alloc && alloc) {
    allocate(alloc);
  } else if (ptr) {
    KUIPER_CHECK(!need_alloc, "need_alloc with an external pointer");
    init_buffer(alloc, data_type_, need_alloc, ptr);
  }
}

void Tensor::init_buffer(std::shared_ptr<base::DeviceAllocator> alloc, base::DataType,
                         bool need_alloc, void* ptr) {
  if (!alloc && !need_alloc) {
    buffer_ = std::make_shared<base::Buffer>(byte_size(), nullptr, ptr, true);
  } else {
    allocate(alloc, true);
  }
}

void Tensor::to_hip(void* stream) {
  KUIPER_CHECK(buffer_ != nullptr, "empty tensor");
  if (buffer_->device_type() == base::DeviceType::kDeviceHIP) return;
  KUIPER_CHECK(buffer_->device_type() == base::DeviceType::kDeviceCPU,
               "to_hip from an unknown device");
  auto alloc = base::HIPDeviceAllocatorFactory::get_instance();
  auto dev = std::make_shared<base::Buffer>(byte_size(), alloc);
  KUIPER_CHECK(dev->ptr() != nullptr, "device allocation failed");
  // Synchronous: the host buffer may be released right after.
  alloc->memcpy(buffer_->ptr(), dev->ptr(), byte_size(), base::MemcpyKind::kMemcpyCPU2CUDA,
                stream, true);
  buffer_ = dev;
}

void Tensor::to_cpu() {
  KUIPER_CHECK(buffer_ != nullptr, "empty tensor");
  if (buffer_->device_type() == base::DeviceType::kDeviceCPU) return;
  auto alloc = base::CPUDeviceAllocatorFactory::get_instance();
  auto host = std::make_shared<base::Buffer>(byte_size(), alloc);
  alloc->memcpy(buffer_->ptr(), host->ptr(), byte_size(), base::MemcpyKind::kMemcpyCUDA2CPU,
                nullptr, true);
  buffer_ = host;
}

bool Tensor::is_empty() const {
  return size_ == 0 || buffer_ == nullptr || buffer_->ptr() == nullptr;
}

void Tensor::reshape(const std::vector<int32_t>& dims) {
  const size_t size = reduce_dims(dims);
  if (!buffer_) {
    dims_ = dims;
    size_ = size;
    return;
  }
  if (size > size_) {
    auto nb = std::make_shared<base::Buffer>(size * base::DataTypeSize(data_type_),
                                             buffer_->allocator());
    KUIPER_CHECK(nb->ptr() != nullptr, "reallocation failed");
    buffer_ = nb;
  }
  dims_ = dims;
  size_ = size;
}

int32_t Tensor::get_dim(int32_t idx) const {
  KUIPER_CHECK(idx >= 0 && idx < static_cast<int32_t>(dims_.size()), "dim index out of range");
  return dims_[idx];
}

std::vector<size_t> Tensor::strides() const {
  std::vector<size_t> s;
  for (size_t i = 0; i + 1 < dims_.size(); ++i)
    s.push_back(reduce_dims(std::vector<int32_t>(dims_.begin() + i + 1, dims_.end())));
  s.push_back(1);
  return s;
}

bool Tensor::assign(std::shared_ptr<base::Buffer> buffer) {
  if (!buffer) return false;
  if (buffer_ && buffer_->device_type() != buffer->device_type()) return false;
  if (byte_size() > buffer->byte_size()) return false;
  buffer_ = buffer;
  return true;
}

void Tensor::reset(base::DataType data_type, const std::vector<int32_t>& dims) {
  data_type_ = data_type;
  dims_ = dims;
  size_ = reduce_dims(dims);
  buffer_ = nullptr;
}

void Tensor::set_device_type(base::DeviceType t) const {
  if (buffer_) buffer_->set_device_type(t);
}

base::DeviceType Tensor::device_type() const {
  return buffer_ ? buffer_->device_type() : base::DeviceType::kDeviceUnknown;
}

bool Tensor::allocate(std::shared_ptr<base::DeviceAllocator> allocator, bool need_realloc) {
  if (!allocator) return false;
  const size_t bytes = byte_size();
  if (!bytes) return false;
  if (buffer_ && bytes <= buffer_->byte_size() && !need_realloc) return true;
  buffer_ = std::make_shared<base::Buffer>(bytes, allocator);
  return buffer_->ptr() != nullptr;
}

Tensor Tensor::clone() const {
  Tensor t = *this;
  KUIPER_CHECK(buffer_ != nullptr, "clone of an empty tensor");
  t.buffer_ = std::make_shared<base::Buffer>(byte_size(), buffer_->allocator());
  KUIPER_CHECK(t.buffer_->ptr() != nullptr, "allocation failed");
  t.buffer_->copy_from(buffer_.get());
  return t;
}

}  // namespace tensor

namespace kernel {
HipConfig::~HipConfig() {
  if (stream) kl_stream_destroy(stream);
}
int HipConfig::create() { return kl_stream_create(&stream); }
}  // namespace kernel
