// neurogrid_gpu.cpp - the C++ restatement of gpu/bindings/gpu.go's wrappers
// for the per-layer kernel path (see neurogrid_gpu.hpp). Each function cites
// the Go wrapper it follows; the error text is the one that wrapper formats.
// Where the Go code would index an empty or short slice and panic (a
// position list that is empty, a shape with too few dimensions for the
// wrapper's shape rule), or hand the kernel a tensor smaller than the call
// reads or writes through it (a device access past the allocation), these
// functions return an error instead.
#include "neurogrid_gpu.hpp"

#include <cstdarg>
#include <cstdio>

#include "bf16_utils.h"
#include "kernels.h"
#include "matmul.h"
#include "memory.h"
#include "quantize.h"

namespace neurogrid {
namespace {

Error Errorf(const char* fmt, ...) {
    char buf[256];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return Error(buf);
}

// A shape with fewer than `rank` dimensions, which the Go wrapper would index
// out of range.
Error ShapeError(const char* what, const Tensor* t, size_t rank) {
    return Errorf("%s: tensor has %zu dimensions, needs at least %zu", what, t->Shape.size(), rank);
}

// A tensor (or position list) with fewer elements than the call touches.
Error SizeError(const char* what, const char* operand, int64_t have, int64_t need) {
    return Errorf("%s: %s has %lld elements, the call needs %lld", what, operand, static_cast<long long>(have),
                  static_cast<long long>(need));
}

}  // namespace

size_t DtypeSize(Dtype d) {  // tensor.go:33-44
    switch (d) {
        case Dtype::FP32: return 4;
        case Dtype::FP16: return 2;
        case Dtype::INT8: return 1;
    }
    return 0;
}

int64_t Tensor::NumElements() const {  // tensor.go:64-71
    int64_t n = 1;
    for (int64_t d : Shape) n *= d;
    return n;
}

int64_t Tensor::ByteSize() const { return NumElements() * static_cast<int64_t>(DtypeSize(Type)); }

Error Tensor::Validate() const {  // tensor.go:94-104
    if (Shape.empty()) return Error("tensor shape cannot be empty");
    for (size_t i = 0; i < Shape.size(); ++i)
        if (Shape[i] <= 0)
            return Errorf("tensor dimension %zu must be positive, got %lld", i, static_cast<long long>(Shape[i]));
    return Error();
}

Tensor NewTensor(std::vector<int64_t> shape, Dtype dtype, int device) {  // tensor.go:50-57
    Tensor t;
    t.Shape = std::move(shape);
    t.Type = dtype;
    t.Device = device;
    return t;
}

// ---------------------------------------------------------------- device management

bool HasCUDA() {  // gpu.go:64-70
    int count = 0;
    if (GetDeviceCount(&count)) return false;
    return count > 0;
}

Error InitGPU(int deviceID) {  // gpu.go:73-79
    const int r = cuda_init(deviceID);
    if (r != 0) return Errorf("CUDA init failed with code %d", r);
    return Error();
}

void ShutdownGPU() { cuda_shutdown(); }  // gpu.go:82-84

Error GetDeviceCount(int* count) {  // gpu.go:87-94
    int n = 0;
    const int r = cuda_get_device_count(&n);
    if (r != 0) return Errorf("failed to get device count: %d", r);
    *count = n;
    return Error();
}

Error SetDevice(int deviceID) {  // gpu.go:97-103
    const int r = cuda_set_device(deviceID);
    if (r != 0) return Errorf("failed to set device %d: code %d", deviceID, r);
    return Error();
}

Error GetDeviceInfo(DeviceInfo* info) {  // gpu.go:106-118
    ::DeviceInfo c{};
    const int r = cuda_get_device_info(&c);
    if (r != 0) return Errorf("failed to get device info: %d", r);
    info->Name = c.name;
    info->Major = c.major;
    info->Minor = c.minor;
    info->TotalMemory = static_cast<uint64_t>(c.total_memory);
    return Error();
}

Error SyncDevice() {  // gpu.go:121-127
    const int r = cuda_sync_device();
    if (r != 0) return Errorf("device sync failed: %d", r);
    return Error();
}

Error GetMemoryUsed(uint64_t* used) {  // gpu.go:130-137
    size_t u = 0;
    const int r = cuda_get_memory_used(&u);
    if (r != 0) return Errorf("failed to get memory usage: %d", r);
    *used = u;
    return Error();
}

// ---------------------------------------------------------------- tensors

Error AllocateTensor(Tensor* t) {  // gpu.go:140-159
    if (t == nullptr) return Error("tensor is nil");
    if (Error e = t->Validate()) return e;
    if (t->Device < 0 || t->Device > 7) return Errorf("invalid device ID: %d", t->Device);
    const size_t size = static_cast<size_t>(t->ByteSize());
    void* p = nullptr;
    const int r = cuda_malloc(&p, size);
    if (r != 0) return Errorf("CUDA malloc failed: %d (size=%zu)", r, size);
    t->Data = p;
    return Error();
}

void FreeTensor(Tensor* t) {  // gpu.go:162-168
    if (t == nullptr || t->Data == nullptr) return;
    cuda_free(t->Data);
    t->Data = nullptr;
}

Error CopyToDevice(Tensor* t, const std::vector<float>& data) {  // gpu.go:171-189
    if (t == nullptr || t->Data == nullptr) return Error("tensor not allocated");
    const int64_t n = t->NumElements();
    if (static_cast<int64_t>(data.size()) < n)
        return Errorf("data size %zu < tensor size %lld", data.size(), static_cast<long long>(n));
    const int r = cuda_copy_to_device(t->Data, data.data(), static_cast<size_t>(n), static_cast<int>(t->Type));
    if (r != 0) return Errorf("copy to device failed: %d", r);
    return Error();
}

Error CopyToHost(std::vector<float>& data, const Tensor* t) {  // gpu.go:192-210
    if (t == nullptr || t->Data == nullptr) return Error("tensor not allocated");
    const int64_t n = t->NumElements();
    if (static_cast<int64_t>(data.size()) < n)
        return Errorf("buffer size %zu < tensor size %lld", data.size(), static_cast<long long>(n));
    const int r = cuda_copy_to_host(data.data(), t->Data, static_cast<size_t>(n), static_cast<int>(t->Type));
    if (r != 0) return Errorf("copy to host failed: %d", r);
    return Error();
}

Error CopyToDeviceINT8(Tensor* t, const std::vector<int8_t>& data) {  // gpu.go:213-233
    if (t == nullptr || t->Data == nullptr) return Error("tensor not allocated");
    if (t->Type != Dtype::INT8) return Error("tensor dtype must be INT8");
    const int64_t n = t->NumElements();
    if (static_cast<int64_t>(data.size()) < n)
        return Errorf("data size %zu < tensor size %lld", data.size(), static_cast<long long>(n));
    const int r = cuda_copy_int8_to_device(t->Data, data.data(), static_cast<size_t>(n));
    if (r != 0) return Errorf("copy INT8 to device failed: %d", r);
    return Error();
}

Error CopyToHostINT8(std::vector<int8_t>& data, const Tensor* t) {  // gpu.go:236-253
    if (t == nullptr || t->Data == nullptr) return Error("tensor not allocated");
    if (t->Type != Dtype::INT8) return Error("tensor dtype must be INT8");
    const int64_t n = t->NumElements();
    if (static_cast<int64_t>(data.size()) < n)
        return Errorf("buffer size %zu < tensor size %lld", data.size(), static_cast<long long>(n));
    const int r = cuda_copy_int8_to_host(data.data(), t->Data, static_cast<size_t>(n));
    if (r != 0) return Errorf("copy INT8 to host failed: %d", r);
    return Error();
}

// ---------------------------------------------------------------- kernels

Error RMSNorm(Tensor* output, const Tensor* input, const Tensor* weight, float eps) {  // gpu.go:256-279
    if (output == nullptr || input == nullptr || weight == nullptr) return Error("nil tensor");
    if (output->Data == nullptr || input->Data == nullptr || weight->Data == nullptr)
        return Error("tensor not allocated");
    if (input->Shape.empty()) return ShapeError("RMSNorm", input, 1);
    const int64_t hidden = input->Shape.back();
    if (hidden <= 0) return Errorf("RMSNorm: hidden size %lld must be positive", static_cast<long long>(hidden));
    const int64_t tokens = input->NumElements() / hidden;
    if (weight->NumElements() < hidden) return SizeError("RMSNorm", "weight", weight->NumElements(), hidden);
    if (output->NumElements() < input->NumElements())
        return SizeError("RMSNorm", "output", output->NumElements(), input->NumElements());
    const int r = cuda_rmsnorm(output->Data, input->Data, weight->Data, static_cast<int>(tokens),
                               static_cast<int>(hidden), eps);
    if (r != 0) return Errorf("RMSNorm failed: %d", r);
    return Error();
}

Error SiLU(Tensor* output, const Tensor* input) {  // gpu.go:282-296
    if (output == nullptr || input == nullptr) return Error("nil tensor");
    if (output->NumElements() < input->NumElements())
        return SizeError("SiLU", "output", output->NumElements(), input->NumElements());
    const int r = cuda_silu(output->Data, input->Data, static_cast<size_t>(input->NumElements()));
    if (r != 0) return Errorf("SiLU failed: %d", r);
    return Error();
}

Error Add(Tensor* c, const Tensor* a, const Tensor* b) {  // gpu.go:299-314
    if (c == nullptr || a == nullptr || b == nullptr) return Error("nil tensor");
    if (b->NumElements() < a->NumElements()) return SizeError("Add", "b", b->NumElements(), a->NumElements());
    if (c->NumElements() < a->NumElements()) return SizeError("Add", "c", c->NumElements(), a->NumElements());
    const int r = cuda_add(c->Data, a->Data, b->Data, static_cast<size_t>(a->NumElements()));
    if (r != 0) return Errorf("Add failed: %d", r);
    return Error();
}

// gpu.go:317-355: [batch, seq, heads, headDim]; the host positions go to a
// temporary device buffer for the call, then cuda_rope (split-half pairs,
// theta 10000). The Go wrapper frees the buffer with a deferred cudaFree,
// which waits for the device; the device is synchronised before the free here.
Error RoPE(Tensor* output, const Tensor* input, const std::vector<int32_t>& positions, int headDim) {
    if (output == nullptr || input == nullptr) return Error("nil tensor");
    if (input->Shape.size() < 4) return Error("input must have 4 dimensions: [batch, seq, heads, head_dim]");
    const int batch = static_cast<int>(input->Shape[0]);
    const int seq = static_cast<int>(input->Shape[1]);
    const int heads = static_cast<int>(input->Shape[2]);
    const int64_t tokens = static_cast<int64_t>(batch) * seq;
    const int64_t touched = tokens * heads * headDim;
    if (static_cast<int64_t>(positions.size()) < tokens)
        return SizeError("RoPE", "positions", static_cast<int64_t>(positions.size()), tokens);
    if (input->NumElements() < touched) return SizeError("RoPE", "input", input->NumElements(), touched);
    if (output->NumElements() < touched) return SizeError("RoPE", "output", output->NumElements(), touched);
    const size_t bytes = positions.size() * sizeof(int32_t);
    void* dpos = nullptr;
    if (cuda_malloc(&dpos, bytes) != 0) return Error("failed to allocate positions on GPU");
    Error err;
    if (positions.empty() || cuda_copy_int8_to_device(dpos, positions.data(), bytes) != 0) {
        err = Error("failed to copy positions to GPU");
    } else {
        const int r = cuda_rope(output->Data, input->Data, static_cast<const int*>(dpos), batch, seq, heads, headDim);
        if (r != 0) err = Errorf("RoPE failed: %d", r);
        (void)cuda_sync_device();
    }
    cuda_free(dpos);
    return err;
}

Error GEMMFP16(Tensor* c, const Tensor* a, const Tensor* b, bool transposeA, bool transposeB) {  // gpu.go:358-392
    if (c == nullptr || a == nullptr || b == nullptr) return Error("nil tensor");
    if (a->Shape.size() < 2) return ShapeError("GEMM FP16", a, 2);
    if (b->Shape.size() < 2) return ShapeError("GEMM FP16", b, 2);
    const int64_t M = transposeA ? a->Shape[1] : a->Shape[0];
    const int64_t K = transposeA ? a->Shape[0] : a->Shape[1];
    const int64_t N = transposeB ? b->Shape[0] : b->Shape[1];
    if (a->NumElements() < M * K) return SizeError("GEMM FP16", "a", a->NumElements(), M * K);
    if (b->NumElements() < K * N) return SizeError("GEMM FP16", "b", b->NumElements(), K * N);
    if (c->NumElements() < M * N) return SizeError("GEMM FP16", "c", c->NumElements(), M * N);
    const int r = cuda_gemm_fp16(c->Data, a->Data, b->Data, static_cast<int>(M), static_cast<int>(K),
                                 static_cast<int>(N), transposeA, transposeB);
    if (r != 0) return Errorf("GEMM FP16 failed: %d", r);
    return Error();
}

Error GEMMINT8(Tensor* c, const Tensor* a, const Tensor* b, const Tensor* scale, bool transposeB) {  // gpu.go:395-424
    if (c == nullptr || a == nullptr || b == nullptr || scale == nullptr) return Error("nil tensor");
    if (a->Shape.size() < 2) return ShapeError("GEMM INT8", a, 2);
    if (b->Shape.size() < 2) return ShapeError("GEMM INT8", b, 2);
    const int64_t M = a->Shape[0], K = a->Shape[1];
    const int64_t N = transposeB ? b->Shape[0] : b->Shape[1];
    if (b->NumElements() < K * N) return SizeError("GEMM INT8", "b", b->NumElements(), K * N);
    if (c->NumElements() < M * N) return SizeError("GEMM INT8", "c", c->NumElements(), M * N);
    if (scale->NumElements() < N) return SizeError("GEMM INT8", "scale", scale->NumElements(), N);
    const int r = cuda_gemm_int8(c->Data, a->Data, b->Data, scale->Data, static_cast<int>(M), static_cast<int>(K),
                                 static_cast<int>(N), transposeB);
    if (r != 0) return Errorf("GEMM INT8 failed: %d", r);
    return Error();
}

Error QuantizePerTensor(Tensor* output, Tensor* scale, const Tensor* input) {  // gpu.go:427-442
    if (output == nullptr || scale == nullptr || input == nullptr) return Error("nil tensor");
    if (output->NumElements() < input->NumElements())
        return SizeError("quantize", "output", output->NumElements(), input->NumElements());
    const int r = cuda_quantize_per_tensor(output->Data, scale->Data, input->Data,
                                           static_cast<size_t>(input->NumElements()));
    if (r != 0) return Errorf("quantize failed: %d", r);
    return Error();
}

Error DequantizePerTensor(Tensor* output, const Tensor* input, const Tensor* scale) {  // gpu.go:445-460
    if (output == nullptr || input == nullptr || scale == nullptr) return Error("nil tensor");
    if (output->NumElements() < input->NumElements())
        return SizeError("dequantize", "output", output->NumElements(), input->NumElements());
    const int r = cuda_dequantize_per_tensor(output->Data, input->Data, scale->Data,
                                             static_cast<size_t>(input->NumElements()));
    if (r != 0) return Errorf("dequantize failed: %d", r);
    return Error();
}

Error QuantizeWeights(Tensor* output, Tensor* scales, const Tensor* input) {  // gpu.go:463-482
    if (output == nullptr || scales == nullptr || input == nullptr) return Error("nil tensor");
    if (input->Shape.size() < 2) return ShapeError("quantize weights", input, 2);
    if (output->NumElements() < input->NumElements())
        return SizeError("quantize weights", "output", output->NumElements(), input->NumElements());
    if (scales->NumElements() < input->Shape[1])
        return SizeError("quantize weights", "scales", scales->NumElements(), input->Shape[1]);
    const int r = cuda_quantize_weights(output->Data, scales->Data, input->Data, static_cast<int>(input->Shape[0]),
                                        static_cast<int>(input->Shape[1]));
    if (r != 0) return Errorf("quantize weights failed: %d", r);
    return Error();
}

Error GatherEmbeddings(void* output, const void* embedTable, const void* dTokenIDs, int hiddenSize,
                       int numTokens) {  // gpu.go:1277-1285
    const int r = cuda_gather_embeddings(output, embedTable, static_cast<const int*>(dTokenIDs), hiddenSize, numTokens);
    if (r != 0) return Errorf("gather embeddings failed: %d", r);
    return Error();
}

// ---------------------------------------------------------------- bf16

Error CheckBF16Support(bool* supported) {  // gpu.go:1329-1336
    int s = 0;
    const int r = cuda_check_bf16_support(&s);
    if (r != 0) return Errorf("failed to check BF16 support: %d", r);
    *supported = s != 0;
    return Error();
}

Error FP16ToBF16(void* output, const void* input, int numElements) {  // gpu.go:1339-1345
    const int r = cuda_fp16_to_bf16(output, input, static_cast<size_t>(numElements));
    if (r != 0) return Errorf("FP16→BF16 failed: %d", r);
    return Error();
}

Error BF16ToFP16(void* output, const void* input, int numElements) {  // gpu.go:1348-1354
    const int r = cuda_bf16_to_fp16(output, input, static_cast<size_t>(numElements));
    if (r != 0) return Errorf("BF16→FP16 failed: %d", r);
    return Error();
}

}  // namespace neurogrid
