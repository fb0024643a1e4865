// neurogrid_gpu.hpp - host-side C++ mirror of the reference's Go bindings for
// the per-layer kernel path, over this library's C ABI.
//
// The reference's Go host reaches libgpu_engine.so through the cgo wrappers
// in gpu/bindings/gpu.go; Go is not available in this build, so these
// functions restate those wrappers in C++: the same names, the same argument
// meaning and shape rules (numTokens = numel / shape[-1], RoPE's
// [batch, seq, heads, headDim], GEMM dimensions from the operands' shapes),
// and the same error text. A Go `error` becomes an `Error` whose message is
// the one gpu.go formats; an empty Error is nil. Functions that return
// (value, error) in Go take an out-parameter and return the Error. Where a Go
// wrapper would panic (a shape with too few dimensions for its shape rule, an
// empty position list) or pass the kernel a tensor smaller than the call
// touches, the C++ one returns an Error before any launch.
//
// Wrappers restated (gpu/bindings/gpu.go): HasCUDA :64, InitGPU :73,
// ShutdownGPU :82, GetDeviceCount :87, SetDevice :97, GetDeviceInfo :106,
// SyncDevice :121, GetMemoryUsed :130, AllocateTensor :140, FreeTensor :162,
// CopyToDevice :171, CopyToHost :192, CopyToDeviceINT8 :213,
// CopyToHostINT8 :236, RMSNorm :256, SiLU :282, Add :299, RoPE :317,
// GEMMFP16 :358, GEMMINT8 :395, QuantizePerTensor :427,
// DequantizePerTensor :445, QuantizeWeights :463, GatherEmbeddings :1277,
// CheckBF16Support :1329, FP16ToBF16 :1339, BF16ToFP16 :1348.
// Tensor and Dtype restate pkg/types/tensor.go:11-104.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace neurogrid {

// Go's `error`: empty is nil.
class Error {
public:
    Error() = default;
    explicit Error(std::string msg) : msg_(std::move(msg)) {}
    explicit operator bool() const { return !msg_.empty(); }
    const std::string& message() const { return msg_; }

private:
    std::string msg_;
};

// pkg/types/tensor.go:11-16; the value is also the copy functions' dtype code.
enum class Dtype : int { FP32 = 0, FP16 = 1, INT8 = 2 };

size_t DtypeSize(Dtype d);  // tensor.go:33-44

// pkg/types/tensor.go:47-104: a device buffer with its shape and dtype.
struct Tensor {
    std::vector<int64_t> Shape;
    Dtype Type = Dtype::FP32;
    int Device = 0;
    void* Data = nullptr;

    int64_t NumElements() const;
    int64_t ByteSize() const;
    Error Validate() const;
};

Tensor NewTensor(std::vector<int64_t> shape, Dtype dtype, int device = 0);

struct DeviceInfo {
    std::string Name;
    int Major = 0;
    int Minor = 0;
    uint64_t TotalMemory = 0;
};

// device management
bool HasCUDA();
Error InitGPU(int deviceID);
void ShutdownGPU();
Error GetDeviceCount(int* count);
Error SetDevice(int deviceID);
Error GetDeviceInfo(DeviceInfo* info);
Error SyncDevice();
Error GetMemoryUsed(uint64_t* used);

// tensors
Error AllocateTensor(Tensor* t);
void FreeTensor(Tensor* t);
Error CopyToDevice(Tensor* t, const std::vector<float>& data);
Error CopyToHost(std::vector<float>& data, const Tensor* t);
Error CopyToDeviceINT8(Tensor* t, const std::vector<int8_t>& data);
Error CopyToHostINT8(std::vector<int8_t>& data, const Tensor* t);

// kernels
Error RMSNorm(Tensor* output, const Tensor* input, const Tensor* weight, float eps);
Error SiLU(Tensor* output, const Tensor* input);
Error Add(Tensor* c, const Tensor* a, const Tensor* b);
Error RoPE(Tensor* output, const Tensor* input, const std::vector<int32_t>& positions, int headDim);
Error GEMMFP16(Tensor* c, const Tensor* a, const Tensor* b, bool transposeA, bool transposeB);
Error GEMMINT8(Tensor* c, const Tensor* a, const Tensor* b, const Tensor* scale, bool transposeB);
Error QuantizePerTensor(Tensor* output, Tensor* scale, const Tensor* input);
Error DequantizePerTensor(Tensor* output, const Tensor* input, const Tensor* scale);
Error QuantizeWeights(Tensor* output, Tensor* scales, const Tensor* input);
Error GatherEmbeddings(void* output, const void* embedTable, const void* dTokenIDs, int hiddenSize, int numTokens);

// bf16
Error CheckBF16Support(bool* supported);
Error FP16ToBF16(void* output, const void* input, int numElements);
Error BF16ToFP16(void* output, const void* input, int numElements);

}  // namespace neurogrid
