// softmax.hip - row softmax over fp16 rows (ABI completeness; not on the
// per-layer path). y_i = RN_f16(exp(x_i - m) / sum_j exp(x_j - m)) with m the
// true row maximum. The reference kernel (gpu/cuda/kernels.cu:580-631) shifts
// by one thread's partial maximum instead; softmax is shift-invariant, so the
// results agree wherever the reference's exponentials do not overflow.
#include "ng_common.hpp"

namespace ng {

constexpr int kSmThreads = 256;

__global__ __launch_bounds__(kSmThreads) void softmax_kernel(uint16_t* out, const uint16_t* in, int cols) {
    __shared__ float s_red[kSmThreads / kWave];
    const size_t off = static_cast<size_t>(blockIdx.x) * cols;
    const uint16_t* x = in + off;
    uint16_t* y = out + off;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;

    float m = -__builtin_inff();
    for (int i = threadIdx.x; i < cols; i += kSmThreads) m = fmaxf(m, to_f32<f16>(x[i]));
    m = wave_max_f32(m);
    if (lane == 0) s_red[wid] = m;
    __syncthreads();
    m = s_red[0];
    for (int j = 1; j < kSmThreads / kWave; ++j) m = fmaxf(m, s_red[j]);
    __syncthreads();

    float s = 0.0f;
    for (int i = threadIdx.x; i < cols; i += kSmThreads) s += expf(to_f32<f16>(x[i]) - m);
    s = wave_sum_f32(s);
    if (lane == 0) s_red[wid] = s;
    __syncthreads();
    s = 0.0f;
    for (int j = 0; j < kSmThreads / kWave; ++j) s += s_red[j];

    for (int i = threadIdx.x; i < cols; i += kSmThreads) y[i] = from_f32<f16>(expf(to_f32<f16>(x[i]) - m) / s);
}

}  // namespace ng

using namespace ng;

extern "C" int cuda_softmax(void* output, const void* input, int num_rows, int row_size) {
    NG_REQUIRE(output && input, "cuda_softmax: null pointer");
    NG_REQUIRE(num_rows > 0 && row_size > 0, "cuda_softmax: num_rows=%d row_size=%d must be > 0", num_rows,
               row_size);
    softmax_kernel<<<dim3(num_rows), dim3(kSmThreads), 0, stream()>>>(static_cast<uint16_t*>(output),
                                                                     static_cast<const uint16_t*>(input), row_size);
    NG_CHECK_LAUNCH("cuda_softmax");
    return 0;
}
