// Buffer and Tensor of the host API (the reference's include/base/buffer.h:6-43
// and include/tensor/tensor.h:12-142), with to_hip() in place of to_cuda().
#pragma once
#include <memory>
#include <vector>

#include "kuiper/alloc.h"
#include "kuiper/base.h"

namespace base {

// Owning (allocated through `allocator`) or external (use_external: the
// memory belongs to someone else, e.g. an mmap'd model file) byte buffer.
class Buffer : public NoCopyable, public std::enable_shared_from_this<Buffer> {
 public:
  explicit Buffer() = default;
  explicit Buffer(size_t byte_size, std::shared_ptr<DeviceAllocator> allocator = nullptr,
                  void* ptr = nullptr, bool use_external = false);
  virtual ~Buffer();
  bool allocate();
  // Copies min(sizes) bytes from `buffer`, picking the copy kind from the
  // two device types.
  void copy_from(const Buffer& buffer) const;
  void copy_from(const Buffer* buffer) const;
  void* ptr() { return ptr_; }
  const void* ptr() const { return ptr_; }
  size_t byte_size() const { return byte_size_; }
  std::shared_ptr<DeviceAllocator> allocator() const { return allocator_; }
  DeviceType device_type() const { return device_type_; }
  void set_device_type(DeviceType device_type) { device_type_ = device_type; }
  std::shared_ptr<Buffer> get_shared_from_this() { return shared_from_this(); }
  bool is_external() const { return use_external_; }

 private:
  size_t byte_size_ = 0;
  void* ptr_ = nullptr;
  bool use_external_ = false;
  DeviceType device_type_ = DeviceType::kDeviceUnknown;
  std::shared_ptr<DeviceAllocator> allocator_;
};

}  // namespace base

namespace tensor {

class Tensor {
 public:
  explicit Tensor() = default;
  explicit Tensor(base::DataType data_type, int32_t dim0, bool need_alloc = false,
                  std::shared_ptr<base::DeviceAllocator> alloc = nullptr, void* ptr = nullptr);
  explicit Tensor(base::DataType data_type, int32_t dim0, int32_t dim1, bool need_alloc = false,
                  std::shared_ptr<base::DeviceAllocator> alloc = nullptr, void* ptr = nullptr);
  explicit Tensor(base::DataType data_type, int32_t dim0, int32_t dim1, int32_t dim2,
                  bool need_alloc = false, std::shared_ptr<base::DeviceAllocator> alloc = nullptr,
                  void* ptr = nullptr);
  explicit Tensor(base::DataType data_type, std::vector<int32_t> dims, bool need_alloc = false,
                  std::shared_ptr<base::DeviceAllocator> alloc = nullptr, void* ptr = nullptr);

  // Moves the data to host memory / to the HIP device (a no-op when it is
  // already there); `stream` is a hipStream_t as void*.
  void to_cpu();
  void to_hip(void* stream = nullptr);

  bool is_empty() const;
  void init_buffer(std::shared_ptr<base::DeviceAllocator> alloc, base::DataType data_type,
                   bool need_alloc, void* ptr);
  template <typename T>
  T* ptr() {
    return buffer_ ? reinterpret_cast<T*>(buffer_->ptr()) : nullptr;
  }
  template <typename T>
  const T* ptr() const {
    return buffer_ ? reinterpret_cast<const T*>(buffer_->ptr()) : nullptr;
  }
  template <typename T>
  T* ptr(int64_t index) {
    KUIPER_CHECK(buffer_ && buffer_->ptr(), "empty tensor");
    return reinterpret_cast<T*>(buffer_->ptr()) + index;
  }
  template <typename T>
  const T* ptr(int64_t index) const {
    KUIPER_CHECK(buffer_ && buffer_->ptr(), "empty tensor");
    return reinterpret_cast<const T*>(buffer_->ptr()) + index;
  }
  // Element access on host memory only.
  template <typename T>
  T& index(int64_t offset) {
    KUIPER_CHECK(offset >= 0 && offset < static_cast<int64_t>(size()), "index out of range");
    KUIPER_CHECK(device_type() == base::DeviceType::kDeviceCPU, "index() needs host memory");
    return *(reinterpret_cast<T*>(buffer_->ptr()) + offset);
  }
  template <typename T>
  const T& index(int64_t offset) const {
    KUIPER_CHECK(offset >= 0 && offset < static_cast<int64_t>(size()), "index out of range");
    KUIPER_CHECK(device_type() == base::DeviceType::kDeviceCPU, "index() needs host memory");
    return *(reinterpret_cast<const T*>(buffer_->ptr()) + offset);
  }

  // Changes the shape; reallocates (without keeping data) when the new size
  // needs more bytes than the buffer holds.
  void reshape(const std::vector<int32_t>& dims);
  std::shared_ptr<base::Buffer> get_buffer() const { return buffer_; }
  size_t size() const { return size_; }
  size_t byte_size() const { return size_ * base::DataTypeSize(data_type_); }
  int32_t dims_size() const { return static_cast<int32_t>(dims_.size()); }
  base::DataType data_type() const { return data_type_; }
  int32_t get_dim(int32_t idx) const;
  const std::vector<int32_t>& dims() const { return dims_; }
  std::vector<size_t> strides() const;
  bool assign(std::shared_ptr<base::Buffer> buffer);
  void reset(base::DataType data_type, const std::vector<int32_t>& dims);
  void set_device_type(base::DeviceType device_type) const;
  base::DeviceType device_type() const;
  bool allocate(std::shared_ptr<base::DeviceAllocator> allocator, bool need_realloc = false);
  Tensor clone() const;

 private:
  size_t size_ = 0;
  std::vector<int32_t> dims_;
  std::shared_ptr<base::Buffer> buffer_;
  base::DataType data_type_ = base::DataType::kDataTypeUnknown;
};

}  // namespace tensor
