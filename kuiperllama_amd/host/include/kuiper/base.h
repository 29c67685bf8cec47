// Base types of the MI355X backend's C++ host API: the same names, values and
// error behaviour as the reference's include/base/base.h:11-150, with one more
// device type, kDeviceHIP, and without the glog dependency (failed checks
// print and abort, as glog's CHECK/LOG(FATAL) do).
#pragma once
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>

namespace model {
// include/base/base.h:12-32
enum class ModelBufferType {
  kInputTokens = 0,
  kInputEmbeddings = 1,
  kOutputRMSNorm = 2,
  kKeyCache = 3,
  kValueCache = 4,
  kQuery = 5,
  kInputPos = 6,
  kScoreStorage = 7,
  kOutputMHA = 8,
  kAttnOutput = 9,
  kW1Output = 10,
  kW2Output = 11,
  kW3Output = 12,
  kFFNRMSNorm = 13,
  kForwardOutput = 15,
  kForwardOutputCPU = 16,
  kSinCache = 17,
  kCosCache = 18,
};
}  // namespace model

namespace base {
// include/base/base.h:36-40 plus the HIP device of this backend.
enum class DeviceType : uint8_t {
  kDeviceUnknown = 0,
  kDeviceCPU = 1,
  kDeviceCUDA = 2,
  kDeviceHIP = 3,
};

enum class DataType : uint8_t {
  kDataTypeUnknown = 0,
  kDataTypeFp32 = 1,
  kDataTypeInt8 = 2,
  kDataTypeInt32 = 3,
};

enum class ModelType : uint8_t {
  kModelTypeUnknown = 0,
  kModelTypeLLama2 = 1,
};

enum class TokenizerType {
  kEncodeUnknown = -1,
  kEncodeSpe = 0,
  kEncodeBpe = 1,
};

inline size_t DataTypeSize(DataType t) {
  switch (t) {
    case DataType::kDataTypeFp32: return sizeof(float);
    case DataType::kDataTypeInt8: return sizeof(int8_t);
    case DataType::kDataTypeInt32: return sizeof(int32_t);
    default: return 0;
  }
}

class NoCopyable {
 protected:
  NoCopyable() = default;
  ~NoCopyable() = default;
  NoCopyable(const NoCopyable&) = delete;
  NoCopyable& operator=(const NoCopyable&) = delete;
};

// include/base/base.h:77-85
enum StatusCode : uint8_t {
  kSuccess = 0,
  kFunctionUnImplement = 1,
  kPathNotValid = 2,
  kModelParseError = 3,
  kInternalError = 5,
  kKeyValueHasExist = 6,
  kInvalidArgument = 7,
};

class Status {
 public:
  Status(int code = StatusCode::kSuccess, std::string err_message = "")
      : code_(code), message_(std::move(err_message)) {}
  Status& operator=(int code) {
    code_ = code;
    return *this;
  }
  bool operator==(int code) const { return code_ == code; }
  bool operator!=(int code) const { return code_ != code; }
  operator int() const { return code_; }
  operator bool() const { return code_ == kSuccess; }
  int32_t get_err_code() const { return code_; }
  const std::string& get_err_msg() const { return message_; }
  void set_err_msg(const std::string& m) { message_ = m; }

 private:
  int code_ = StatusCode::kSuccess;
  std::string message_;
};

namespace error {
Status Success(const std::string& err_msg = "");
Status FunctionNotImplement(const std::string& err_msg = "");
Status PathNotValid(const std::string& err_msg = "");
Status ModelParseError(const std::string& err_msg = "");
Status InternalError(const std::string& err_msg = "");
Status KeyHasExits(const std::string& err_msg = "");
Status InvalidArgument(const std::string& err_msg = "");
}  // namespace error

[[noreturn]] void fatal(const char* file, int line, const std::string& what);

}  // namespace base

// A failed precondition aborts with a message (the reference's glog CHECK).
#define KUIPER_CHECK(cond, msg)                                                     \
  do {                                                                              \
    if (!(cond)) ::base::fatal(__FILE__, __LINE__, std::string("check failed: ") + \
                                                       #cond + " " + (msg));        \
  } while (0)

// include/base/base.h:123-134: a failed Status is fatal.
#define STATUS_CHECK(call)                                                              \
  do {                                                                                  \
    const ::base::Status& status_ = (call);                                             \
    if (!status_)                                                                       \
      ::base::fatal(__FILE__, __LINE__,                                                 \
                    "Infer error, code " + std::to_string(int(status_)) + ": " +        \
                        status_.get_err_msg());                                         \
  } while (0)
