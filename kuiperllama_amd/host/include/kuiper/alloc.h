// Device allocators (the reference's include/base/alloc.h:7-92): a CPU
// allocator and the HIP allocator of this backend, which replaces
// CUDADeviceAllocator.  Device memory, copies and fills go through the C ABI
// of libkuiper_hip (include/kuiper_hip.h); this header has no HIP dependency.
#pragma once
#include <map>
#include <memory>
#include <vector>

#include "kuiper/base.h"

namespace base {

// include/base/alloc.h:7-12; the CUDA enumerators stand for "device" here.
enum class MemcpyKind {
  kMemcpyCPU2CPU = 0,
  kMemcpyCPU2CUDA = 1,
  kMemcpyCUDA2CPU = 2,
  kMemcpyCUDA2CUDA = 3,
};

class DeviceAllocator {
 public:
  explicit DeviceAllocator(DeviceType device_type) : device_type_(device_type) {}
  virtual ~DeviceAllocator() = default;
  virtual DeviceType device_type() const { return device_type_; }
  virtual void release(void* ptr) const = 0;
  virtual void* allocate(size_t byte_size) const = 0;
  // Copies byte_size bytes; `stream` is a hipStream_t (as void*) or null.
  virtual void memcpy(const void* src_ptr, void* dest_ptr, size_t byte_size,
                      MemcpyKind memcpy_kind = MemcpyKind::kMemcpyCPU2CPU, void* stream = nullptr,
                      bool need_sync = false) const;
  virtual void memset_zero(void* ptr, size_t byte_size, void* stream, bool need_sync = false);

 private:
  DeviceType device_type_ = DeviceType::kDeviceUnknown;
};

class CPUDeviceAllocator : public DeviceAllocator {
 public:
  CPUDeviceAllocator();
  void* allocate(size_t byte_size) const override;
  void release(void* ptr) const override;
};

// A reusable block of the HIP allocator's pool.
struct HipMemoryBuffer {
  void* data = nullptr;
  size_t byte_size = 0;
  bool busy = false;
};

// Pooled device allocator (the reference policy of source/base/alloc_cu.cpp:7-112):
// requests above 1 MiB reuse the best-fitting free big block whose size is
// within 1 MiB of the request; smaller requests reuse the first free small
// block that fits; a released small block stays pooled until more than 1 GiB
// of small blocks sits idle on the device, then the idle ones are freed.
// Not thread-safe (the reference's allocator is not either).
class HIPDeviceAllocator : public DeviceAllocator {
 public:
  HIPDeviceAllocator();
  void* allocate(size_t byte_size) const override;
  void release(void* ptr) const override;
  // Bytes currently held from the device (busy and pooled).
  size_t pooled_bytes() const;

 private:
  mutable std::map<int, size_t> idle_small_bytes_;
  mutable std::map<int, std::vector<HipMemoryBuffer>> big_buffers_;
  mutable std::map<int, std::vector<HipMemoryBuffer>> small_buffers_;
};

class CPUDeviceAllocatorFactory {
 public:
  static std::shared_ptr<CPUDeviceAllocator> get_instance();
};

class HIPDeviceAllocatorFactory {
 public:
  static std::shared_ptr<HIPDeviceAllocator> get_instance();
};

// The allocator for a device type (CPU or HIP); null for others.
std::shared_ptr<DeviceAllocator> allocator_for(DeviceType device_type);

}  // namespace base
