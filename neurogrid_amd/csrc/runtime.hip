// runtime.hip - device management, transfers and the launch stream
// (memory.h, stream.h, cuda_check_bf16_support).
//
// Reference: gpu/cuda/memory.cu:32-223 and gpu/cuda/stream.cu:4-12. The
// dtype-converting copies (fp32 on the host, fp16 on the device) convert on
// the host for up to 64 K elements and move the 16-bit data with one
// synchronous hipMemcpy. Larger copies move fp32 through a device buffer of
// at most 16 MiB, chunk by chunk, and convert on the device, as the reference
// does with one buffer of the whole size (memory.cu:145-213).
#include "ng_common.hpp"
#include "../../include/memory.h"

#include <algorithm>
#include <atomic>
#include <string.h>
#include <vector>

namespace ng {

static std::atomic<hipStream_t> g_stream{nullptr};
static bool g_initialized = false;
static int g_current_device = 0;

int device_cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cache[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

// fp32 -> binary16, round to nearest even (subnormals, overflow to inf, NaN kept quiet).
static uint16_t f32_to_f16_bits(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return static_cast<uint16_t>(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);  // >= 65520: rounds to inf
    if (ax < 0x33000000u) return static_cast<uint16_t>(sign);             // < 2^-25: rounds to 0
    const int e = static_cast<int>(ax >> 23) - 127;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    if (e < -14) {
        const int shift = -1 - e;  // value = m 2^(e-23), subnormal unit 2^-24
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return static_cast<uint16_t>(sign | q);
    }
    uint32_t q = (static_cast<uint32_t>(e + 15) << 10) | ((m >> 13) & 0x3ffu);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return static_cast<uint16_t>(sign | q);
}

// binary16 -> fp32, exact.
static float f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            float v = static_cast<float>(m) * 0x1p-24f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

// Device halves of the converting copies, bit for bit the host conversions
// above: fp32 -> fp16 rounds to nearest even (v_cvt_f16_f32) and gives NaN
// as sign | 0x7e00; fp16 -> fp32 is exact and keeps a NaN's payload (the
// hardware conversion would set its quiet bit).
__global__ __launch_bounds__(256) void copy_f32_to_f16_kernel(uint16_t* out, const float* in, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * 256;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
        const float v = in[i];
        const uint32_t x = __builtin_bit_cast(uint32_t, v);
        out[i] = (x & 0x7fffffffu) > 0x7f800000u ? static_cast<uint16_t>(((x >> 16) & 0x8000u) | 0x7e00u)
                                                : from_f32<f16>(v);
    }
}

__global__ __launch_bounds__(256) void copy_f16_to_f32_kernel(float* out, const uint16_t* in, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * 256;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
        const uint32_t h = in[i];
        out[i] = (h & 0x7c00u) == 0x7c00u && (h & 0x3ffu) != 0
                     ? __builtin_bit_cast(float, ((h & 0x8000u) << 16) | 0x7f800000u | ((h & 0x3ffu) << 13))
                     : to_f32<f16>(static_cast<uint16_t>(h));
    }
}

// Copies of more than this many elements convert on the device. Measured on
// MI355X (fp32 from pageable host memory): 16 M values took 29 ms to the
// device converted on the host, 2.5 ms staged and converted on the device;
// 64 K took 0.14 ms either way, and 1 K 13 us on the host against 25 us.
constexpr size_t kDeviceConvertMin = size_t(1) << 16;
constexpr size_t kConvertChunk = size_t(1) << 22;  // elements per staged chunk: 16 MiB of fp32

static unsigned copy_blocks(size_t n) { return static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 4096)); }

// fp32 host -> fp16 device through a device buffer. The launch stream orders
// each chunk's conversion after the copies and kernels before it, and is
// synchronised before the buffer takes the next chunk.
static int copy_f32_to_f16_staged(uint16_t* dst, const float* src, size_t n) {
    const size_t chunk = std::min(n, kConvertChunk);
    float* tmp = nullptr;
    NG_HIP_CHECK(hipMalloc(&tmp, chunk * sizeof(float)));
    const hipStream_t s = stream();
    hipError_t e = hipSuccess;
    for (size_t off = 0; off < n && e == hipSuccess; off += chunk) {
        const size_t m = std::min(chunk, n - off);
        e = hipMemcpy(tmp, src + off, m * sizeof(float), hipMemcpyHostToDevice);
        if (e != hipSuccess) break;
        copy_f32_to_f16_kernel<<<dim3(copy_blocks(m)), dim3(256), 0, s>>>(dst + off, tmp, m);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(s);
    }
    (void)hipFree(tmp);
    NG_HIP_CHECK(e);
    return 0;
}

// fp16 device -> fp32 host through a device buffer, chunk by chunk.
static int copy_f16_to_f32_staged(float* dst, const uint16_t* src, size_t n) {
    const size_t chunk = std::min(n, kConvertChunk);
    float* tmp = nullptr;
    NG_HIP_CHECK(hipMalloc(&tmp, chunk * sizeof(float)));
    const hipStream_t s = stream();
    hipError_t e = hipSuccess;
    for (size_t off = 0; off < n && e == hipSuccess; off += chunk) {
        const size_t m = std::min(chunk, n - off);
        copy_f16_to_f32_kernel<<<dim3(copy_blocks(m)), dim3(256), 0, s>>>(tmp, src + off, m);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e == hipSuccess) e = hipMemcpy(dst + off, tmp, m * sizeof(float), hipMemcpyDeviceToHost);
    }
    (void)hipFree(tmp);
    NG_HIP_CHECK(e);
    return 0;
}

}  // namespace ng

using namespace ng;

extern "C" hipStream_t ng_get_stream(void) { return g_stream.load(std::memory_order_acquire); }
extern "C" void ng_set_stream(hipStream_t s) { g_stream.store(s, std::memory_order_release); }

extern "C" int cuda_init(int device_id) {
    if (g_initialized) return 0;
    int count = 0;
    NG_HIP_CHECK(hipGetDeviceCount(&count));
    NG_REQUIRE(device_id >= 0 && device_id < count, "Invalid device ID %d (available: 0-%d)", device_id, count - 1);
    NG_HIP_CHECK(hipSetDevice(device_id));
    g_current_device = device_id;
    g_initialized = true;
    void* dummy = nullptr;
    NG_HIP_CHECK(hipMalloc(&dummy, 1024));
    NG_HIP_CHECK(hipFree(dummy));
    return gemm_scratch_init(device_id);
}

extern "C" void cuda_shutdown(void) {
    if (g_initialized) {
        (void)hipDeviceSynchronize();
        (void)hipGetLastError();
        gemm_release();
        (void)hipDeviceReset();
        g_initialized = false;
    }
}

extern "C" int cuda_get_device_count(int* count) {
    NG_REQUIRE(count, "cuda_get_device_count: null pointer");
    NG_HIP_CHECK(hipGetDeviceCount(count));
    return 0;
}

extern "C" int cuda_set_device(int device_id) {
    NG_HIP_CHECK(hipSetDevice(device_id));
    g_current_device = device_id;
    // Look up this device's copy of the allocation-free GEMM's scratch array
    // now, outside any stream capture, rather than on its first call there.
    return gemm_scratch_init(device_id);
}

extern "C" int cuda_get_device_info(DeviceInfo* info) {
    NG_REQUIRE(info, "cuda_get_device_info: null pointer");
    hipDeviceProp_t prop;
    NG_HIP_CHECK(hipGetDeviceProperties(&prop, g_current_device));
    strncpy(info->name, prop.name, 255);
    info->name[255] = '\0';
    info->major = prop.major;
    info->minor = prop.minor;
    info->total_memory = prop.totalGlobalMem;
    return 0;
}

extern "C" int cuda_sync_device(void) {
    NG_HIP_CHECK(hipDeviceSynchronize());
    return 0;
}

extern "C" int cuda_get_memory_used(size_t* used) {
    NG_REQUIRE(used, "cuda_get_memory_used: null pointer");
    size_t free_mem = 0, total_mem = 0;
    NG_HIP_CHECK(hipMemGetInfo(&free_mem, &total_mem));
    *used = total_mem - free_mem;
    return 0;
}

extern "C" int cuda_malloc(void** ptr, size_t size) {
    NG_REQUIRE(ptr, "cuda_malloc: null pointer");
    if (size == 0) {
        *ptr = nullptr;
        return 0;
    }
    NG_HIP_CHECK(hipMalloc(ptr, size));
    return 0;
}

extern "C" void cuda_free(void* ptr) {
    if (ptr != nullptr) (void)hipFree(ptr);
}

extern "C" int cuda_copy_to_device(void* dst, const void* src, size_t n, int dtype) {
    NG_REQUIRE(dtype >= 0 && dtype <= 2, "cuda_copy_to_device: unknown dtype %d", dtype);
    if (n == 0) return 0;
    NG_REQUIRE(dst && src, "cuda_copy_to_device: null pointer");
    if (dtype == 0) {
        NG_HIP_CHECK(hipMemcpy(dst, src, n * sizeof(float), hipMemcpyHostToDevice));
    } else if (dtype == 1) {
        if (n > kDeviceConvertMin)
            return copy_f32_to_f16_staged(static_cast<uint16_t*>(dst), static_cast<const float*>(src), n);
        std::vector<uint16_t> tmp(n);
        const float* s = static_cast<const float*>(src);
        for (size_t i = 0; i < n; ++i) tmp[i] = f32_to_f16_bits(s[i]);
        NG_HIP_CHECK(hipMemcpy(dst, tmp.data(), n * sizeof(uint16_t), hipMemcpyHostToDevice));
    } else {
        NG_HIP_CHECK(hipMemcpy(dst, src, n, hipMemcpyHostToDevice));
    }
    return 0;
}

extern "C" int cuda_copy_to_host(void* dst, const void* src, size_t n, int dtype) {
    NG_REQUIRE(dtype >= 0 && dtype <= 2, "cuda_copy_to_host: unknown dtype %d", dtype);
    if (n == 0) return 0;
    NG_REQUIRE(dst && src, "cuda_copy_to_host: null pointer");
    if (dtype == 0) {
        NG_HIP_CHECK(hipMemcpy(dst, src, n * sizeof(float), hipMemcpyDeviceToHost));
    } else if (dtype == 1) {
        if (n > kDeviceConvertMin)
            return copy_f16_to_f32_staged(static_cast<float*>(dst), static_cast<const uint16_t*>(src), n);
        std::vector<uint16_t> tmp(n);
        NG_HIP_CHECK(hipMemcpy(tmp.data(), src, n * sizeof(uint16_t), hipMemcpyDeviceToHost));
        float* d = static_cast<float*>(dst);
        for (size_t i = 0; i < n; ++i) d[i] = f16_bits_to_f32(tmp[i]);
    } else {
        NG_HIP_CHECK(hipMemcpy(dst, src, n, hipMemcpyDeviceToHost));
    }
    return 0;
}

extern "C" int cuda_copy_int8_to_device(void* dst, const void* src, size_t n) {
    if (n == 0) return 0;
    NG_REQUIRE(dst && src, "cuda_copy_int8_to_device: null pointer");
    NG_HIP_CHECK(hipMemcpy(dst, src, n, hipMemcpyHostToDevice));
    return 0;
}

extern "C" int cuda_copy_int8_to_host(void* dst, const void* src, size_t n) {
    if (n == 0) return 0;
    NG_REQUIRE(dst && src, "cuda_copy_int8_to_host: null pointer");
    NG_HIP_CHECK(hipMemcpy(dst, src, n, hipMemcpyDeviceToHost));
    return 0;
}

extern "C" int cuda_check_bf16_support(int* supported) {
    NG_REQUIRE(supported, "cuda_check_bf16_support: null pointer");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        *supported = 0;
        return -1;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        *supported = 0;
        return -1;
    }
    // Every gfx9 CDNA device from gfx90a on, and gfx11/gfx12, has bf16 conversions.
    const char* arch = prop.gcnArchName;
    *supported = (strncmp(arch, "gfx90a", 6) == 0 || strncmp(arch, "gfx94", 5) == 0 ||
                  strncmp(arch, "gfx95", 5) == 0 || strncmp(arch, "gfx11", 5) == 0 ||
                  strncmp(arch, "gfx12", 5) == 0)
                     ? 1
                     : 0;
    return 0;
}

extern "C" const char* ng_version(void) { return "neurogrid-amd 0.1.0 (gfx950)"; }
