// matmul.hip - cuda_gemm_int8 and cuda_gemm_fp16 for gfx950.
//
// Reference: gpu/cuda/matmul.cu:75-156 (cuda_gemm_fp16: cublasHgemm with the
// row-major -> column-major operand swap) and :169-244 (cuda_gemm_int8:
// cudaMalloc a K*N fp16 copy, dequantize_and_copy, cuda_gemm_fp16, cudaFree).
//
// Weight-streaming path (transpose_b, M <= 128). The engine's INT8 layers call
// cuda_gemm_int8 with B stored [N, K] and one scale per row of B
// (layer.cu:487-501,551,575). For up to a few hundred tokens the product is
// bound by reading B once, 1 byte per weight; the reference moves 5 (read
// int8, write fp16, read fp16). Here the kernel reads the codes, turns them
// into exact fp16 integers in registers and feeds the matrix cores:
//   C[m, n] = fp16( scale[n] * sum_k A[m, k] * q[n, k] )
// with the sum in fp32 (every product of an fp16 activation and an integer
// code in [-128, 127] is exact in fp32). The reference rounds q * scale to
// fp16 first and sums those; the two differ by at most 2^-11 of
// sum_k |A[m, k] * q[n, k] * scale[n]| plus the accumulation error.
//
// Three kernels, by M, K and N (see gemm_i8w):
//   M <= 2, and M <= 4 with K, N < 8192: gemv_i8w_kernel, dot-product
//       instructions, each load reads 1 KiB contiguous of one row of B;
//   4 < M <= 16 with K, N < 8192: gemm_i8w_kernel, matrix cores, A read from
//       L2, waves split K within the block;
//   otherwise, up to M = 128: gemm_i8w_split_kernel, matrix cores, A staged
//       in LDS, K split between wave groups of a block and between blocks
//       (slices whose sums a second kernel adds), A cut into token tiles
//       for few rows of B.
// Above 128 rows of A (prefill) the product is bound by the matrix cores:
// gemm_i8w_prefill_kernel, a tiled GEMM whose B tiles are converted on their
// way into LDS (see the prefill section); from 4096 rows on (kLtMinM) the
// reference's composition through hipBLASLt, which is faster there. B stored
// [K, N] always goes through the composition (dequantize, then hipBLASLt).
// Each fused kernel also has a shared form (ng_gemm_int8_shared_a) that runs
// several products with the same A and the same launch shape in one launch,
// each product's blocks as in its own launch; the GEMV kernel's shared form
// can also normalise A itself (ng_rmsnorm_gemm_int8_shared_a and the add +
// RMSNorm form), each block in registers, for the decode steps norm -> q/k/v.
// MFMA layout: v_mfma_f32_16x16x32_f16 multiplies a 16 x 32 tile of A (rows
// m) by a 32 x 16 tile of B^T (columns n). Lane l supplies row (l % 16) of
// each operand and 8 values of k; the accumulator lane l holds rows
// 4 * (l / 16) + i, column l % 16. In a chunk of 64 k, lane group g = l / 16
// holds k = 16g .. 16g + 15 of its row of B (16 codes); the first 8 feed one
// MFMA and the last 8 another, and A's lanes take the same k, so each MFMA
// sums matching k. The two MFMA kernels read B in whole 128-byte lines (8 rows
// x 128 codes per load instruction) and reorder the codes into that layout
// through LDS: loading straight into it reads 64 bytes per row per
// instruction, which streams about 25% slower on MI355X.
// Every sum is taken in a fixed order (partial sums meet in LDS or in the
// slice buffer, never through atomics), so results do not depend on timing.
#include "ng_common.hpp"
#include "ng_exact.hpp"
#include "../../include/kernels.h"
#include "../../include/matmul.h"
#include "../../include/neurogrid_ext.h"

#include <hipblaslt/hipblaslt.h>

#include <atomic>
#include <climits>
#include <map>
#include <mutex>
#include <set>
#include <tuple>
#include <utility>
#include <vector>

// Partial sums of the allocation-free entry point (ng_gemm_int8_noalloc): a
// device array of fixed size that every GPU the library runs on holds until
// the process ends. In host code `scratch` names a host-side stand-in, not
// device memory: its device address is looked up once per device
// (hipGetSymbolAddress, see scratch_ptr) and only that address is used.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

namespace ng {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;          // K granularity of the MFMA kernels (one 16x16x32 MFMA pair per lane group)
constexpr int kMaxFusedM = 128;     // rows of A the weight-streaming path takes

// Two int8 codes (bytes SEL0 and SEL1 of one dword) -> two exact fp16 values.
// The bytes are biased to u = q + 128, placed under an fp16 exponent of 2^10
// with v_perm (fp16 bits 0x6400 | u = 1024 + u), and 1152 is subtracted in
// fp16: every step is exact.
template <uint32_t SEL>
__device__ __forceinline__ uint32_t codes_to_f16x2(uint32_t w) {
    const f16x2 bias = {static_cast<f16>(-1152.0f), static_cast<f16>(-1152.0f)};
    const f16x2 v = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, w ^ 0x80808080u, SEL)) + bias;
    return __builtin_bit_cast(uint32_t, v);
}

// A dword as two fp16 values. Takes the dword by value: __builtin_bit_cast
// applied directly to an ext_vector element (v[i]) reads element 0.
__device__ __forceinline__ f16x2 as_f16x2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }

// 16 codes of one row of B -> the B operands of two MFMAs (codes 0-7, 8-15).
__device__ __forceinline__ void codes16_to_operands(const u32x4 v, f16x8& b0, f16x8& b1) {
    const u32x4 x = {codes_to_f16x2<0x04010400u>(v[0]), codes_to_f16x2<0x04030402u>(v[0]),
                     codes_to_f16x2<0x04010400u>(v[1]), codes_to_f16x2<0x04030402u>(v[1])};
    const u32x4 y = {codes_to_f16x2<0x04010400u>(v[2]), codes_to_f16x2<0x04030402u>(v[2]),
                     codes_to_f16x2<0x04010400u>(v[3]), codes_to_f16x2<0x04030402u>(v[3])};
    b0 = __builtin_bit_cast(f16x8, x);
    b1 = __builtin_bit_cast(f16x8, y);
}

// MT tiles of 16 rows of A x one tile of 16 rows of B per block. The WAVES
// waves split K in 128-k batches (batch b goes to wave b % WAVES); each loads
// U batches, then multiplies them, and the waves' partial sums are added
// through LDS in wave order. B is read in whole 128-byte lines (8 rows x 128
// codes per instruction) and reordered into the MFMA layout through a per-wave
// LDS buffer, as in the split kernel below.
//
// Products that share A (ng_gemm_int8_shared_a) run in one launch of the
// *_shared_kernel forms of this kernel and of the GEMV kernel below: blocks
// first[p] .. first[p + 1] - 1 run product p exactly as the blocks 0 .. of its
// own launch would, so each C is bit-identical to its own call. A product's
// pointers are picked with selects, not by indexing the argument arrays
// (which would copy them to scratch memory).
constexpr int kMaxShared = 4;
struct SharedSet {
    uint16_t* c[kMaxShared];
    const int8_t* b[kMaxShared];
    const float* scale[kMaxShared];
    int n[kMaxShared];
    int first[kMaxShared];  // first block of each product, increasing; INT_MAX past the last
};

// Per-product split-K parameters (gemm_i8w_split_shared_kernel): the
// product's partial-sum region, its slice count, tiles of B, batches per
// slice and token tiles.
struct SplitSet {
    float* part[kMaxShared];
    int S[kMaxShared];
    int tiles[kMaxShared];
    int cps[kMaxShared];
    int TT[kMaxShared];
};

// Element p of four (a select chain on a wave-uniform p).
template <typename V>
__device__ __forceinline__ V pick4(int p, V v0, V v1, V v2, V v3) {
    return p == 0 ? v0 : p == 1 ? v1 : p == 2 ? v2 : v3;
}

// Runs block(c, b, scale, n, block index within the product, p) for the
// product p that owns this block.
template <typename F>
__device__ __forceinline__ void shared_dispatch(const SharedSet& s, F&& block) {
    const int blk = blockIdx.x;
    const int p = (blk >= s.first[1]) + (blk >= s.first[2]) + (blk >= s.first[3]);
    block(pick4(p, s.c[0], s.c[1], s.c[2], s.c[3]), pick4(p, s.b[0], s.b[1], s.b[2], s.b[3]),
          pick4(p, s.scale[0], s.scale[1], s.scale[2], s.scale[3]), pick4(p, s.n[0], s.n[1], s.n[2], s.n[3]),
          blk - pick4(p, s.first[0], s.first[1], s.first[2], s.first[3]), p);
}

template <int MT, int NT, int WAVES, int U>
__device__ __forceinline__ void gemm_i8w_block(uint16_t* __restrict__ c, const uint16_t* __restrict__ a,
                                               const int8_t* __restrict__ b, const float* __restrict__ scale,
                                               int M, int N, int K, int blk) {
    static_assert(NT == 1, "one tile of B per block");
    __shared__ f32x4 partial[WAVES - 1][MT][kWave];
    __shared__ __align__(16) u32x4 lds_b[WAVES][2 * kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int col = lane & 15;
    const int grp = lane >> 4;
    const int n0 = blk * 16;
    const int nbatch = (K + 127) / 128;
    const bool half_last = (K % 128) != 0;

    const int8_t* brow[2];
    int bpiece[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int r = 8 * j + (lane >> 3);
        bpiece[j] = (lane & 7) ^ (r >> 1);
        brow[j] = b + static_cast<size_t>(min(n0 + r, N - 1)) * K;
    }
    const uint16_t* ap[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) ap[t] = a + static_cast<size_t>(min(16 * t + col, M - 1)) * K + 16 * grp;

    f32x4 acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int cnt = wave < nbatch ? (nbatch - wave + WAVES - 1) / WAVES : 0;
    if (cnt > 0) {
        const int last = wave + (cnt - 1) * WAVES;
        u32x4 bv[U][2];
        u32x4 av[U][MT][2][2];
        auto load = [&](int slot, int i) {
            // Batches past this wave's last are clamped to it (and skipped in multiply).
            const int bt = min(wave + i * WAVES, last);
            const bool half = half_last && bt == nbatch - 1;
            const size_t kb = static_cast<size_t>(bt) * 128;
#pragma unroll
            for (int j = 0; j < 2; ++j) bv[slot][j] = ld16_stream(brow[j] + kb + 16 * (half ? (bpiece[j] & 3) : bpiece[j]));
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const size_t k = kb + ((half && st == 1) ? 0 : 64 * st);
                    av[slot][t][st][0] = ld16(ap[t] + k);
                    av[slot][t][st][1] = ld16(ap[t] + k + 8);
                }
        };
        auto multiply = [&](int u, int i) {
            const int bt = wave + i * WAVES;
            const bool past = i >= cnt;
            const bool half = half_last && bt == nbatch - 1;
            lds_b[wave][lane] = bv[u][0];
            lds_b[wave][kWave + lane] = bv[u][1];
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                // A batch past this wave's last, and the second half of a half
                // batch, hold reloaded codes and activations: skipped (an inf
                // activation times a zero code would give NaN).
                if (past || (half && st == 1)) continue;
                const int p = 4 * st + grp;
                const u32x4 v = lds_b[wave][8 * col + (p ^ (col >> 1))];
                f16x8 b0, b1;
                codes16_to_operands(v, b0, b1);
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av[u][t][st][0]), b0,
                                                                    acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av[u][t][st][1]), b1,
                                                                    acc[t], 0, 0, 0);
                }
            }
            __builtin_amdgcn_wave_barrier();
        };
        for (int i = 0; i < cnt; i += U) {
#pragma unroll
            for (int u = 0; u < U; ++u) load(u, i + u);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < U; ++u) multiply(u, i + u);
        }
    }

    if (wave > 0) {
#pragma unroll
        for (int i = 0; i < MT; ++i) partial[wave - 1][i][lane] = acc[i];
    }
    __syncthreads();
    if (wave != 0) return;
    const int n = n0 + col;
    const float s = scale[min(n, N - 1)];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        f32x4 v = acc[i];
#pragma unroll
        for (int w = 0; w < WAVES - 1; ++w) v += partial[w][i][lane];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int m = 16 * i + 4 * grp + e;
            if (m < M && n < N) c[static_cast<size_t>(m) * N + n] = from_f32<f16>(v[e] * s);
        }
    }
}

template <int MT, int NT, int WAVES, int U>
__global__ __launch_bounds__(WAVES * kWave) void gemm_i8w_kernel(uint16_t* __restrict__ c,
                                                                  const uint16_t* __restrict__ a,
                                                                  const int8_t* __restrict__ b,
                                                                  const float* __restrict__ scale, int M, int N,
                                                                  int K) {
    gemm_i8w_block<MT, NT, WAVES, U>(c, a, b, scale, M, N, K, blockIdx.x);
}

template <int MT, int NT, int WAVES, int U>
__global__ __launch_bounds__(WAVES * kWave) void gemm_i8w_shared_kernel(SharedSet s, const uint16_t* __restrict__ a,
                                                                         int M, int K) {
    shared_dispatch(s, [&](uint16_t* c, const int8_t* b, const float* scale, int n, int blk, int) {
        gemm_i8w_block<MT, NT, WAVES, U>(c, a, b, scale, M, n, K, blk);
    });
}

template <int MT, int NT, int WAVES, int U>
int launch_i8w(uint16_t* c, const uint16_t* a, const int8_t* b, const float* scale, int M, int N, int K) {
    const unsigned blocks = static_cast<unsigned>((N + 16 * NT - 1) / (16 * NT));
    gemm_i8w_kernel<MT, NT, WAVES, U>
        <<<dim3(blocks), dim3(WAVES * kWave), 0, stream()>>>(c, a, b, scale, M, N, K);
    NG_CHECK_LAUNCH("cuda_gemm_int8");
    return 0;
}

// ---- GEMV-shaped variant (M <= 4) -------------------------------------------
// With one to four rows of A the MFMA layout costs a 16-byte load of A per
// 16 codes in every lane and reads 64 bytes per row of B per instruction.
// Here lane l of a wave takes codes [16l, 16l + 16) of a 1024-code segment, so
// each load instruction reads 1 KiB contiguous of one row of B; the lane's A
// values for that segment are loaded once and reused for R rows. Products are
// summed with v_dot2_f32_f16 (pairs of fp16 products, fp32 sums); the block's
// waves take different segments, and the 256 partial sums of each output are
// added through LDS in a fixed order.
constexpr int kGvWaves = 4;
constexpr int kGvSeg = 1024;  // codes per wave step: 64 lanes x 16

// The products of one 1024-code segment in one lane: R rows of B (codes
// bv[r]) against the lane's 16 values of each of MR rows of A (av[m]). Lanes
// past K pass zeros in both operands: an inf activation times a zero code
// would give NaN.
template <int MR, int R>
__device__ __forceinline__ void gemv_segment(float (&acc)[R][MR], u32x4 (&av)[MR][2], const u32x4 (&bv)[R],
                                             bool kin) {
    if (!kin) {
#pragma unroll
        for (int m = 0; m < MR; ++m) av[m][0] = av[m][1] = u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const u32x4 q = kin ? bv[r] : u32x4{0u, 0u, 0u, 0u};
        f16x8 w0, w1;
        codes16_to_operands(q, w0, w1);
        const u32x4 wl = __builtin_bit_cast(u32x4, w0), wh = __builtin_bit_cast(u32x4, w1);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float s = acc[r][m];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s = __builtin_amdgcn_fdot2(as_f16x2(av[m][0][j]), as_f16x2(wl[j]), s, false);
                s = __builtin_amdgcn_fdot2(as_f16x2(av[m][1][j]), as_f16x2(wh[j]), s, false);
            }
            acc[r][m] = s;
        }
    }
}

// The block's sums: output o = r * MR + m adds red[(w * V + o) * 64 + l] over
// waves w and lanes l; kParts threads add 256 / kParts values each, then one
// thread adds the parts, both in a fixed order. Thread o < V returns output
// o's sum (others 0). The reduction buffer is free again after a barrier.
template <int MR, int R>
__device__ __forceinline__ float gemv_reduce(const float (&acc)[R][MR]) {
    constexpr int V = R * MR;                 // outputs per block
    constexpr int kParts = kGvWaves * kWave / V;  // threads that share one output in the first reduction stage
    static_assert(kGvWaves * kWave % V == 0 && kWave % kParts == 0, "reduction shape");
    __shared__ float red[kGvWaves * V * kWave];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) red[(wave * V + r * MR + m) * kWave + lane] = acc[r][m];
    __syncthreads();
    const int o = tid % V;
    const int part = tid / V;
    constexpr int kPerPart = kGvWaves * kWave / kParts;  // values summed by one thread
    float sum = 0.0f;
#pragma unroll 4
    for (int j = 0; j < kPerPart; ++j) {
        const int idx = part * kPerPart + j;  // (wave, lane) pair
        sum += red[((idx / kWave) * V + o) * kWave + idx % kWave];
    }
    __syncthreads();
    red[o * kParts + part] = sum;
    __syncthreads();
    float v = 0.0f;
    if (tid < V)
        for (int q = 0; q < kParts; ++q) v += red[tid * kParts + q];
    return v;
}

// C = fp16(sum * scale) for the block's rows n0 .. n0 + R - 1 of B.
template <int MR, int R>
__device__ __forceinline__ void gemv_finish(const float (&acc)[R][MR], uint16_t* __restrict__ c,
                                            const float* __restrict__ scale, int M, int N, int n0) {
    const float v = gemv_reduce<MR, R>(acc);
    const int tid = threadIdx.x;
    if (tid < R * MR) {
        const int r = tid / MR, m = tid % MR, n = n0 + r;
        if (m < M && n < N) c[static_cast<size_t>(m) * N + n] = from_f32<f16>(v * scale[n]);
    }
}

// One lane's sums of the GEMV kernels' block for rows n0 .. n0 + R - 1 of B.
template <int MR, int R>
__device__ __forceinline__ void gemv_i8w_sums(float (&acc)[R][MR], const uint16_t* __restrict__ a,
                                              const int8_t* __restrict__ b, int M, int N, int K, int n0) {
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int nseg = (K + kGvSeg - 1) / kGvSeg;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[r][m] = 0.0f;

    for (int sg = wave; sg < nseg; sg += kGvWaves) {
        const int k = sg * kGvSeg + 16 * lane;
        const bool kin = k < K;           // the last segment may end early (K % 16 == 0)
        const int kc = kin ? k : K - 16;  // lanes past K load the last codes and multiply zeros
        u32x4 av[MR][2];
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const uint16_t* ar = a + static_cast<size_t>(min(m, M - 1)) * K + kc;
            av[m][0] = ld16(ar);
            av[m][1] = ld16(ar + 8);
        }
        u32x4 bv[R];
#pragma unroll
        for (int r = 0; r < R; ++r) bv[r] = ld16_stream(b + static_cast<size_t>(min(n0 + r, N - 1)) * K + kc);
        __builtin_amdgcn_sched_barrier(0);
        gemv_segment<MR, R>(acc, av, bv, kin);
    }
}

// One block of the GEMV kernels: rows blk R .. blk R + R - 1 of B.
template <int MR, int R>
__device__ __forceinline__ void gemv_i8w_block(uint16_t* __restrict__ c, const uint16_t* __restrict__ a,
                                               const int8_t* __restrict__ b, const float* __restrict__ scale,
                                               int M, int N, int K, int blk) {
    float acc[R][MR];
    gemv_i8w_sums<MR, R>(acc, a, b, M, N, K, blk * R);
    gemv_finish<MR, R>(acc, c, scale, M, N, blk * R);
}

template <int MR, int R>
__global__ __launch_bounds__(kGvWaves * kWave) void gemv_i8w_kernel(uint16_t* __restrict__ c,
                                                                    const uint16_t* __restrict__ a,
                                                                    const int8_t* __restrict__ b,
                                                                    const float* __restrict__ scale, int M, int N,
                                                                    int K) {
    gemv_i8w_block<MR, R>(c, a, b, scale, M, N, K, blockIdx.x);
}

template <int MR, int R>
__global__ __launch_bounds__(kGvWaves * kWave) void gemv_i8w_shared_kernel(SharedSet s, const uint16_t* __restrict__ a,
                                                                           int M, int K) {
    shared_dispatch(s, [&](uint16_t* c, const int8_t* b, const float* scale, int n, int blk, int) {
        gemv_i8w_block<MR, R>(c, a, b, scale, M, n, K, blk);
    });
}

// gate/up and SwiGLU in one launch (ng_gemm_int8_silu_mul): block blk runs
// the GEMV kernel's block blk of the gate product and of the up product (the
// same R rows of each, both against one load of A), reduces each exactly as
// that block does, and writes gate = fp16(sum * scale), up likewise, and
// out = fp16(silu(gate) * up) with the element-wise kernel's expression. out
// may be gate or up itself: each element is written by one thread, out last.
struct SwigluArgs {
    uint16_t* out;
    uint16_t* gate;
    uint16_t* up;
    const int8_t* bg;
    const int8_t* bu;
    const float* sg;
    const float* su;
};

template <int MR, int R>
__global__ __launch_bounds__(kGvWaves * kWave) void gemv_i8w_swiglu_kernel(SwigluArgs sa, const uint16_t* __restrict__ a,
                                                                           int M, int N, int K) {
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int n0 = blockIdx.x * R;
    const int nseg = (K + kGvSeg - 1) / kGvSeg;
    float accg[R][MR], accu[R][MR];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) accg[r][m] = accu[r][m] = 0.0f;
    for (int sg = wave; sg < nseg; sg += kGvWaves) {
        const int k = sg * kGvSeg + 16 * lane;
        const bool kin = k < K;
        const int kc = kin ? k : K - 16;
        u32x4 av[MR][2];
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const uint16_t* ar = a + static_cast<size_t>(min(m, M - 1)) * K + kc;
            av[m][0] = ld16(ar);
            av[m][1] = ld16(ar + 8);
        }
        u32x4 bvg[R], bvu[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const size_t row = static_cast<size_t>(min(n0 + r, N - 1)) * K + kc;
            bvg[r] = ld16_stream(sa.bg + row);
            bvu[r] = ld16_stream(sa.bu + row);
        }
        __builtin_amdgcn_sched_barrier(0);
        gemv_segment<MR, R>(accg, av, bvg, kin);
        gemv_segment<MR, R>(accu, av, bvu, kin);
    }
    const float vg = gemv_reduce<MR, R>(accg);
    __syncthreads();  // the reduction buffer is reused
    const float vu = gemv_reduce<MR, R>(accu);
    if (tid < R * MR) {
        const int r = tid / MR, m = tid % MR, n = n0 + r;
        if (m < M && n < N) {
            const size_t o = static_cast<size_t>(m) * N + n;
            const uint16_t g = from_f32<f16>(vg * sa.sg[n]), u = from_f32<f16>(vu * sa.su[n]);
            sa.gate[o] = g;
            sa.up[o] = u;
            sa.out[o] = from_f32<f16>(swiglu_f32(to_f32<f16>(g), to_f32<f16>(u)));
        }
    }
}

// A product and the residual add after it (ng_gemm_int8_add): the GEMV
// kernel's blocks, then out = fp16(c + residual) on the rounded product, as
// cuda_add computes it. out may be c or the residual itself: each element is
// written by one thread, out last.
template <int MR, int R>
__global__ __launch_bounds__(kGvWaves * kWave) void gemv_i8w_add_kernel(uint16_t* out, uint16_t* c,
                                                                        const uint16_t* res,
                                                                        const uint16_t* __restrict__ a,
                                                                        const int8_t* __restrict__ b,
                                                                        const float* __restrict__ scale, int M,
                                                                        int N, int K) {
    const int n0 = blockIdx.x * R;
    float acc[R][MR];
    gemv_i8w_sums<MR, R>(acc, a, b, M, N, K, n0);
    const float v = gemv_reduce<MR, R>(acc);
    const int tid = threadIdx.x;
    if (tid < R * MR) {
        const int r = tid / MR, m = tid % MR, n = n0 + r;
        if (m < M && n < N) {
            const size_t o = static_cast<size_t>(m) * N + n;
            const uint16_t cv = from_f32<f16>(v * scale[n]);
            const float sum = to_f32<f16>(cv) + to_f32<f16>(res[o]);
            c[o] = cv;
            out[o] = from_f32<f16>(sum);
        }
    }
}

// RMSNorm (or residual add + RMSNorm) folded into the shared GEMV launch
// (ng_rmsnorm_gemm_int8_shared_a, ng_add_rmsnorm_gemm_int8_shared_a), for
// M <= 2 rows of K <= 8192. Every block normalises the rows itself, and each
// thread normalises exactly the 16-value pieces of A that its lane multiplies
// in the GEMV (segment sg = wave + 4 s, values 16 lane .. 16 lane + 15), so A
// stays in registers: the thread loads its pieces of x (and the residual) and
// of the norm weight, then its rows of B, and the row statistic (one block
// barrier for all rows) and the scaling run while the codes are in flight.
// Each block gets cuda_rmsnorm's (cuda_add_rmsnorm's) bits: the statistic is
// the sum of squares rounded once to fp32 (fp64 sums resolved with their
// error bound, else exact limb sums), which does not depend on the order of
// summation, and the scaling is the same expression. The products are the
// GEMV block's own segment and reduction code, so C is bit-identical too. The
// first block of the launch stores the normalised rows (and the residual sums).
struct NormArgs {
    const uint16_t* x;
    const uint16_t* res;  // residual input (ADD)
    const uint16_t* w;    // norm weight [K]
    uint16_t* normed;     // [M, K]
    uint16_t* res_out;    // [M, K] (ADD)
    float eps;
};

// Row m's exact statistic from the limb sums of the whole row, read from
// memory by every thread of the block (the fast path's rare fallback; the
// decision is uniform over the block).
template <bool ADD>
__device__ __noinline__ float norm_row_ss_exact(const NormArgs& na, int m, int K) {
    constexpr int kT = kGvWaves * kWave;
    __shared__ double s_limb[kGvWaves][3];
    __shared__ int s_flag[kGvWaves];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
    const uint16_t* xr = na.x + static_cast<size_t>(m) * K;
    const uint16_t* rr = ADD ? na.res + static_cast<size_t>(m) * K : nullptr;
    Limbs Lm{0.0, 0.0, 0.0, 0};
    for (int vi = tid; vi < K / 8; vi += kT) {
        float fx[8];
        unpack8<f16>(ld16(xr + vi * 8), fx);
        if (ADD) {
            float fr[8];
            unpack8<f16>(ld16(rr + vi * 8), fr);
#pragma unroll
            for (int i = 0; i < 8; ++i) fx[i] = fx[i] + fr[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) limbs_add(Lm, fx[i]);
    }
    double t = wave_sum_f64_dpp(Lm.t), u = wave_sum_f64_dpp(Lm.u), w = wave_sum_f64_dpp(Lm.w);
    int bad = static_cast<int>(wave_max_u32_dpp(static_cast<uint32_t>(Lm.bad)));
    __syncthreads();  // a previous row's readers are done with s_limb
    if (lane == 0) {
        s_limb[wid][0] = t;
        s_limb[wid][1] = u;
        s_limb[wid][2] = w;
        s_flag[wid] = bad;
    }
    __syncthreads();
    t = u = w = 0.0;
    bad = 0;
    for (int j = 0; j < kGvWaves; ++j) {
        t += s_limb[j][0];
        u += s_limb[j][1];
        w += s_limb[j][2];
        bad |= s_flag[j];
    }
    return bad ? -1.0f : limbs_to_f32(t, u, w);
}

// One block of the fused kernels: the rows of A normalised in registers, then
// the products of the GEMV kernel's block blk (rows blk R .. blk R + R - 1 of
// B), exactly as that block computes them. SEGS: the most 1024-value segments
// of K one wave takes (K <= 4096 SEGS).
// RoPE on two of the products (ng_rmsnorm_qkv_rope_int8): split-half pairs
// (i, i + D/2) of each head of D values, as cuda_rope_with_theta style 0,
// for the tokens' positions.
constexpr int kRopeEpiMaxHalf = 128;  // D <= 256
struct RopeEpi {
    const int* pos;  // [M]
    int D;
    int half;  // D / 2
    int bph;   // blocks per head: half / 4
    float inv_freq[kRopeEpiMaxHalf];
};

template <int MR, int R, int SEGS, bool ADD, bool ROPE = false>
__device__ __forceinline__ void gemv_i8w_norm_block(uint16_t* __restrict__ c, const int8_t* __restrict__ b,
                                                    const float* __restrict__ scale, const NormArgs& na, int M,
                                                    int N, int K, int blk, bool store, bool rope = false,
                                                    const RopeEpi* re = nullptr) {
    static_assert(!ROPE || R == 8, "a RoPE block holds four rotation pairs");
    __shared__ double s_part[kGvWaves][MR];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int n0 = blk * R;
    const int nseg = (K + kGvSeg - 1) / kGvSeg;
    // Row of B (and of C) in slot r: n0 + r, or for a rotated product the
    // block's four pairs of one head, rows h D + q + r (r < 4) and
    // h D + D/2 + q + r - 4. An output's sums do not depend on its slot, so
    // each row gets the GEMV kernel's bits either way.
    // The geometry is read whether or not this product rotates: a read under
    // the product's flag put a branch and a scalar-load wait before every code
    // load.
    const bool rot = ROPE && rope;
    const int rbph = ROPE ? re->bph : 1, rD = ROPE ? re->D : 0, rhalf = ROPE ? re->half : 0;
    const int rh = rot ? blk / rbph : 0;
    const int rq = rot ? (blk - rh * rbph) * 4 : 0;
    const int lo = rot ? rh * rD + rq : n0;              // slots 0 .. 3: rows lo + r
    const int hi = rot ? rh * rD + rhalf + rq - 4 : n0;  // slots 4 .. 7: rows hi + r
    const auto row_of = [&](int r) { return (r < 4 ? lo : hi) + r; };

    // Loads: the lane's pieces of x (res) and w, then its rows of B. They are
    // issued without branches, so that waiting for the first ones does not
    // wait for the codes: a wave with no segment s (sg >= nseg) has every lane
    // past K, at K - 16, and its loads of that segment hit one line per row.
    bool kin[SEGS];
    int kc[SEGS];
    u32x4 xv[SEGS][MR][2], rv[SEGS][MR][2], wv[SEGS][2], bv[SEGS][R];
#pragma unroll
    for (int s = 0; s < SEGS; ++s) {
        const int k = (wave + s * kGvWaves) * kGvSeg + 16 * lane;
        kin[s] = k < K;
        kc[s] = kin[s] ? k : K - 16;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const size_t off = static_cast<size_t>(min(m, M - 1)) * K + kc[s];
            xv[s][m][0] = ld16(na.x + off);
            xv[s][m][1] = ld16(na.x + off + 8);
            if (ADD) {
                rv[s][m][0] = ld16(na.res + off);
                rv[s][m][1] = ld16(na.res + off + 8);
            }
        }
        wv[s][0] = ld16(na.w + kc[s]);
        wv[s][1] = ld16(na.w + kc[s] + 8);
    }
#pragma unroll
    for (int s = 0; s < SEGS; ++s)
#pragma unroll
        for (int r = 0; r < R; ++r)
            bv[s][r] = ld16_stream(b + static_cast<size_t>(min(row_of(r), N - 1)) * K + kc[s]);
    __builtin_amdgcn_sched_barrier(0);

    // o = x, or the rounded sum x + res; squares of x, or of the unrounded
    // fp32 sum, as the row kernels take them. Lanes past K add nothing.
    double ssq[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) ssq[m] = 0.0;
#pragma unroll
    for (int s = 0; s < SEGS; ++s) {
        if (wave + s * kGvWaves >= nseg) continue;
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float s0, s1;
                    if (ADD) {
                        s0 = el_add<f16, 0>(xv[s][m][h][i], rv[s][m][h][i]);
                        s1 = el_add<f16, 1>(xv[s][m][h][i], rv[s][m][h][i]);
                        xv[s][m][h][i] = pack2<f16>(s0, s1);
                    } else {
                        s0 = el_get<f16, 0>(xv[s][m][h][i]);
                        s1 = el_get<f16, 1>(xv[s][m][h][i]);
                    }
                    const double d0 = kin[s] ? static_cast<double>(s0) : 0.0;
                    const double d1 = kin[s] ? static_cast<double>(s1) : 0.0;
                    ssq[m] = __builtin_fma(d0, d0, ssq[m]);
                    ssq[m] = __builtin_fma(d1, d1, ssq[m]);
                }
    }
    if (ADD && store) {
#pragma unroll
        for (int s = 0; s < SEGS; ++s)
#pragma unroll
            for (int m = 0; m < MR; ++m)
                if (kin[s] && m < M) {
                    uint16_t* ro = na.res_out + static_cast<size_t>(m) * K + kc[s];
                    st16(ro, xv[s][m][0]);
                    st16(ro + 8, xv[s][m][1]);
                }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const double S = wave_sum_f64_dpp(ssq[m]);
        if (lane == 0) s_part[wave][m] = S;
    }
    __syncthreads();
    float rs[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        double S = s_part[0][m];
        for (int j = 1; j < kGvWaves; ++j) S += s_part[j][m];
        // Tree height: 16 SEGS terms in one lane, 6 across the wave, 3 across the waves.
        float ss;
        if (!ss_fast_resolve(S, 16 * SEGS + 10, ss)) {
            const float e = norm_row_ss_exact<ADD>(na, min(m, M - 1), K);
            if (e >= 0.0f) ss = e;
        }
        rs[m] = 1.0f / __builtin_sqrtf(ss / static_cast<float>(K) + na.eps);
    }

    // y = RN_f16(RN(o * r) * w): the GEMV's A, in registers.
    float acc[R][MR];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[r][m] = 0.0f;
#pragma unroll
    for (int s = 0; s < SEGS; ++s) {
        if (wave + s * kGvWaves >= nseg) continue;
        u32x4 av[MR][2];
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    av[m][h][i] = pack2<f16>(el_mul<f16, 0>(wv[s][h][i], el_mul<f16, 0>(xv[s][m][h][i], rs[m])),
                                             el_mul<f16, 1>(wv[s][h][i], el_mul<f16, 1>(xv[s][m][h][i], rs[m])));
        if (store) {
#pragma unroll
            for (int m = 0; m < MR; ++m)
                if (kin[s] && m < M) {
                    uint16_t* yo = na.normed + static_cast<size_t>(m) * K + kc[s];
                    st16(yo, av[m][0]);
                    st16(yo + 8, av[m][1]);
                }
        }
        gemv_segment<MR, R>(acc, av, bv[s], kin[s]);
    }
    if (!rot) {
        gemv_finish<MR, R>(acc, c, scale, M, N, n0);
        return;
    }
    // Rotated product: C = fp16(sum * scale) as the GEMV kernel rounds it, then
    // RoPE on the rounded pair, with cuda_rope_with_theta's angle, sincosf and
    // expression, rounded once more. Slot r's partner is r ^ 4 (thread
    // tid ^ 4 MR, in the first wave).
    constexpr int V = R * MR;
    const float v = gemv_reduce<MR, R>(acc);
    float x = 0.0f;
    int r = 0, m = 0, row = 0;
    if (tid < V) {
        r = tid / MR;
        m = tid % MR;
        row = row_of(r);
        x = to_f32<f16>(from_f32<f16>(v * scale[row]));
    }
    const float xp = __shfl_xor(x, 4 * MR, kWave);
    if (tid < V && m < M) {
        float sn, cs;
        sincosf(static_cast<float>(re->pos[m]) * re->inv_freq[rq + (r & 3)], &sn, &cs);
        const float y = r < 4 ? x * cs - xp * sn : xp * sn + x * cs;
        c[static_cast<size_t>(m) * N + row] = from_f32<f16>(y);
    }
}

template <int MR, int R, int SEGS, bool ADD>
__global__ __launch_bounds__(kGvWaves * kWave) void gemv_i8w_norm_shared_kernel(SharedSet s, NormArgs na, int M,
                                                                                int K) {
    shared_dispatch(s, [&](uint16_t* c, const int8_t* b, const float* scale, int n, int blk, int) {
        gemv_i8w_norm_block<MR, R, SEGS, ADD>(c, b, scale, na, M, n, K, blk, blockIdx.x == 0);
    });
}

// The same with RoPE on products 0 and 1 (q and k).
template <int MR, int SEGS>
__global__ __launch_bounds__(kGvWaves * kWave) void gemv_i8w_norm_rope_shared_kernel(SharedSet s, NormArgs na,
                                                                                     RopeEpi re, int M, int K) {
    shared_dispatch(s, [&](uint16_t* c, const int8_t* b, const float* scale, int n, int blk, int p) {
        gemv_i8w_norm_block<MR, 8, SEGS, false, true>(c, b, scale, na, M, n, K, blk, blockIdx.x == 0, p < 2, &re);
    });
}

template <int MR, int R>
int launch_gemv_shared(const SharedSet& set, int blocks, const uint16_t* a, int M, int K) {
    gemv_i8w_shared_kernel<MR, R><<<dim3(static_cast<unsigned>(blocks)), dim3(kGvWaves * kWave), 0, stream()>>>(
        set, a, M, K);
    NG_CHECK_LAUNCH("ng_gemm_int8_shared_a");
    return 0;
}

// Longest rows the fused norm kernels take: two segments per wave.
constexpr int kNormSharedMaxK = 2 * kGvWaves * kGvSeg;
// Most GEMV blocks of a fused norm launch. The fused kernel holds more
// registers than the GEMV kernel (5 waves per SIMD against 8 at one row):
// where the launch fits the GPU in about one round of blocks, folding the
// norm in saves its launch and its latency; with more blocks the launch is
// bound by the codes in flight, and the two calls are faster (measured on
// MI355X at Mistral-7B: q/k/v, 768 blocks, 7.2 against 8.3 us at one token;
// gate/up, 3584 blocks, 23.1 against 21.8 us). Only the GEMV shapes of one
// and two rows (8 rows of B per block) are folded: with four rows the fused
// kernel was slower at every block count measured (TinyLlama's q/k/v, 640
// blocks, 3 rows: 7.9 against 6.4 us).
constexpr int kNormSharedMaxBlocks = 1024;

template <int MR, int R, bool ADD>
int launch_gemv_norm_shared(const SharedSet& set, int blocks, const NormArgs& na, int M, int K) {
    const dim3 grid(static_cast<unsigned>(blocks)), block(kGvWaves * kWave);
    if (K <= kGvWaves * kGvSeg)
        gemv_i8w_norm_shared_kernel<MR, R, 1, ADD><<<grid, block, 0, stream()>>>(set, na, M, K);
    else
        gemv_i8w_norm_shared_kernel<MR, R, 2, ADD><<<grid, block, 0, stream()>>>(set, na, M, K);
    NG_CHECK_LAUNCH(ADD ? "ng_add_rmsnorm_gemm_int8_shared_a" : "ng_rmsnorm_gemm_int8_shared_a");
    return 0;
}

template <int MR, int R>
int launch_gemv(uint16_t* c, const uint16_t* a, const int8_t* b, const float* scale, int M, int N, int K) {
    const unsigned blocks = static_cast<unsigned>((N + R - 1) / R);
    gemv_i8w_kernel<MR, R><<<dim3(blocks), dim3(kGvWaves * kWave), 0, stream()>>>(c, a, b, scale, M, N, K);
    NG_CHECK_LAUNCH("cuda_gemm_int8");
    return 0;
}

// ---- split-K variant --------------------------------------------------------
// For more than a few rows of A the kernel above reads A from L2 once per
// 16 rows of B: at M = 64 that is 8 bytes of A per weight byte. Here a block
// of W waves owns 16 W rows of B and one of S slices of K; the A columns of
// each 128-k batch are staged once in LDS and shared by the block's waves
// (2M / (16 W) bytes of A per weight byte). W = 4, or 8 for K >= 8192 (the
// down projection: 22.5 vs 25.2 us at M = 64, 34.5 vs 40.1 us at M = 128;
// 8 waves were slower at K = 4096, and 2 slower everywhere but N = 1024).
//
// B is read in whole 128-byte lines: each load instruction of a wave covers
// 8 rows x 128 codes (8 lanes per row), two instructions a wave's 16 rows.
// Loading B straight into the MFMA layout instead (4 lanes per row, 64 bytes
// per row per instruction) streams about 25% slower on MI355X. The codes
// reach the MFMA layout through a per-wave LDS buffer: piece p (16 codes) of
// row r sits in slot 8r + (p xor r / 2), so the writes are contiguous and the
// reads conflict-free. (LDS on MI355X serves 256 bytes per clock from 64
// banks. Measured with access-pattern probes, 16-byte reads are conflict-free
// when the rows 0-7 of one lane group and the rows 8-15 of another fall in
// opposite halves of the banks; (p + r / 2) mod 8 breaks that and took two
// clocks per 16 lanes.)
//
// K is divided among blocks and inside them. The G groups of W waves of a
// block take turns of G consecutive batches (group g the batch g of each
// turn), each group with its own LDS copy of its batch of A; at the end the
// groups' sums are added through LDS in group order. With S > 1 each block
// stores those sums in `part` [S][M][N] and a second kernel adds the S slices
// in slice order. Either way the result does not depend on timing. (Having
// the last block of each tile add the slices instead needs an agent-scope
// release and acquire per block, which on MI355X write back and invalidate
// the whole L2: measured 3-5x slower.) Groups inside the block replace slices
// where there are enough tiles to fill the GPU with one slice: no partial
// sums in memory and no second launch.
constexpr int kBatch = 128;  // k per batch

// SW (ng_gemm_int8_silu_mul, one K slice, no token tiles): the block's first
// W/2 waves of each group take rows of the gate product and the last W/2 the
// same rows of the up product (8 W row pairs per block instead of 16 W rows of
// one product). A wave's sums depend only on its own 16 rows of B, which start
// at a multiple of 16 either way, so gate and up are the values of their own
// launches; the up waves hand their rounded values to the gate waves through
// LDS, which write gate, up and fp16(silu(gate) * up).
template <int MT, int W, int G, bool SW = false>
__device__ __forceinline__ void gemm_i8w_split_block(
    uint16_t* __restrict__ c, const uint16_t* __restrict__ a, const int8_t* __restrict__ b,
    const float* __restrict__ scale, float* __restrict__ part, int M, int N, int K, int S, int tiles, int cps,
    int TT, int blk, const SwigluArgs* sw = nullptr) {
    static_assert(!SW || W % 2 == 0, "SW splits the waves of a group in two");
    // A batch of A in LDS. From 4 tiles of A on: 256 bytes per row, 16-byte
    // piece q of row m stored at piece q xor (m mod 16), so the MFMA reads
    // (16 rows, one piece each per lane group) are conflict-free; padded rows
    // (16, 32 or 64 bytes) leave two-way conflicts, unpadded unswizzled rows
    // eight-way ones. With 1 or 2 tiles the rows are padded by 32 bytes
    // instead: measured 6% faster there (gate/up at M = 17-32), while the
    // swizzle is 2-11% faster at M = 64-128.
    constexpr bool kSwizzleA = MT >= 4;
    constexpr int kRowBytes = kSwizzleA ? kBatch * 2 : kBatch * 2 + 32;
    constexpr int kPieces = 16 * MT * 16;       // 16-byte pieces of A per batch
    constexpr int kThreads = G * W * kWave;
    static_assert((G * kPieces) % kThreads == 0, "A pieces must divide among the threads");
    static_assert(G == 1 || (G - 1) * W * MT * kWave * 16 <= 2 * G * 16 * MT * kRowBytes,
                  "the groups' sums must fit in the A buffers");
    __shared__ __align__(16) uint8_t lds_a[2][G][16 * MT * kRowBytes];
    __shared__ __align__(16) u32x4 lds_b[G * W][2 * kWave];

    // With TT > 1 token tiles, block b takes rows 16 MT ty .. of A for unit u
    // (a tile and slice), with the TT blocks of a unit on one XCD (ids u + 8 j
    // apart), so that they read its rows of B from one L2.
    int unit = blk, ty = 0;
    if (TT > 1) {
        const int i = blk / 8;
        ty = i % TT;
        unit = (i / TT) * 8 + blk % 8;
        if (unit >= tiles * S) return;
    }
    const int Mall = M;
    {
        const int m0 = 16 * MT * ty;
        a += static_cast<size_t>(m0) * K;
        c += static_cast<size_t>(m0) * N;
        part += static_cast<size_t>(m0) * N;
        M = min(16 * MT, M - m0);
    }
    const int sl = unit % S;
    const int tile = unit / S;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int kg = wave / W;   // this wave's group: batch kg of each turn
    const int wv = wave % W;   // and its tile of 16 rows of B
    const int col = lane & 15;
    const int grp = lane >> 4;
    const int nbatch = (K + kBatch - 1) / kBatch;  // the last batch holds 64 k when K % 128 == 64
    const bool half_last = (K % kBatch) != 0;
    const int c0 = sl * cps;
    const int c1 = min(c0 + cps, nbatch);
    const bool upw = SW && wv >= W / 2;  // SW: this wave takes the up product's rows
    const int nw = SW ? tile * (8 * W) + 16 * (wv % (W / 2)) : tile * (16 * W) + 16 * wv;  // first row of B
    const int n = nw + col;                                 // row of B this lane multiplies
    if constexpr (SW) {
        b = upw ? sw->bu : sw->bg;
        scale = upw ? sw->su : sw->sg;
    }

    // A and B are read with buffer loads: B from this wave's first row (rows
    // past N clamp to the last one), A from its start, so that per-load
    // offsets are 32-bit instead of 64-bit addresses (2-6% faster at
    // M = 64-128). Offsets are below 16 K bytes for B and 2 M K bytes for A.
    const int nbase = min(nw, N - 1);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(b + static_cast<size_t>(nbase) * K), 0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a), 0, 0x7fffffff,
                                                                        0x00020000);
    uint32_t boff[2];
    int bpiece[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int r = 8 * j + (lane >> 3);
        bpiece[j] = (lane & 7) ^ (r >> 1);
        boff[j] = static_cast<uint32_t>((min(nw + r, N - 1) - nbase) * K);
    }
    constexpr int kP = G * kPieces / kThreads;
    uint32_t aoff[kP];
#pragma unroll
    for (int j = 0; j < kP; ++j) {
        const int pc = (j * kThreads + tid) % kPieces;
        aoff[j] = static_cast<uint32_t>(min(pc / 16, M - 1) * K * 2);
    }

    f32x4 acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Turns, two in flight: the loads of turn i + 1 (B into registers, A
    // into registers on their way to LDS) are issued before turn i is
    // multiplied; A alternates between two LDS buffers, so one barrier per
    // turn separates a buffer's writes from its reads and from its reuse two
    // turns later. A turn starting at batch `first` holds batches first ..
    // first + G - 1; those past the slice load its last batch (every load
    // stays unconditional) and are skipped by multiply.
    // A first: staging it into LDS then waits only for A, not for B.
    auto load = [&](u32x4 (&bv)[2], u32x4 (&ar)[kP], int first) {
#pragma unroll
        for (int j = 0; j < kP; ++j) {
            const int pc = j * kThreads + tid;
            const int cb = min(first + pc / kPieces, c1 - 1);
            const size_t kb = static_cast<size_t>(cb) * kBatch;
            int q = pc % 16;
            if (half_last && cb == nbatch - 1) q &= 7;  // k past K: load the batch's first 64 k again
            ar[j] = __builtin_amdgcn_raw_buffer_load_b128(ra, aoff[j] + static_cast<uint32_t>((kb + 8 * q) * 2), 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep A's loads ahead of B's
        // Pieces 4-7 of a half batch would lie past K: they load pieces 0-3
        // again (and are skipped by multiply).
        const int cb = min(first + kg, c1 - 1);
        const bool half = half_last && cb == nbatch - 1;
        const size_t kb = static_cast<size_t>(cb) * kBatch;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int pcs = half ? (bpiece[j] & 3) : bpiece[j];
            bv[j] = __builtin_amdgcn_raw_buffer_load_b128(rb, boff[j] + static_cast<uint32_t>(kb + 16 * pcs), 0, 2);
        }
    };
    auto stage = [&](int buf, const u32x4 (&ar)[kP]) {
#pragma unroll
        for (int j = 0; j < kP; ++j) {
            const int pc = j * kThreads + tid;
            const int g = pc / kPieces;
            const int row = (pc % kPieces) / 16;
            *reinterpret_cast<u32x4*>(lds_a[buf][g] + row * kRowBytes + 16 * (kSwizzleA ? (pc % 16) ^ (row & 15) : pc % 16)) = ar[j];
        }
    };
    auto multiply = [&](int buf, const u32x4 (&bv)[2], int first) {
        // This wave's codes into the MFMA layout. LDS operations of one wave
        // complete in order, so the reads see the writes, and the next batch's
        // writes come after these reads.
        lds_b[wave][lane] = bv[0];
        lds_b[wave][kWave + lane] = bv[1];
        __builtin_amdgcn_wave_barrier();
        const int cb = first + kg;
        const bool past = cb >= c1;                               // clamped batch: skipped
        const bool half = half_last && cb == nbatch - 1;          // its second 64 k lie past K
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            // A clamped batch, and the second half of a half batch, hold
            // reloaded codes and activations: skipped (wave-uniform), so that
            // an inf activation never meets a padding code (inf * 0 = NaN).
            if (past || (half && st == 1)) continue;
            const int p = 4 * st + grp;
            const u32x4 v = lds_b[wave][8 * col + (p ^ (col >> 1))];
            f16x8 b0, b1;
            codes16_to_operands(v, b0, b1);
            // All tiles' first halves, then their second halves: consecutive
            // MFMAs update different accumulators (2-4% faster at M = 64-128).
            u32x4 a0[MT], a1[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                // pieces 8 st + 2 grp and the next one of row 16 t + col
                const uint8_t* ap = lds_a[buf][kg] + (16 * t + col) * kRowBytes;
                const int q0 = 8 * st + 2 * grp;
                a0[t] = *reinterpret_cast<const u32x4*>(ap + 16 * (kSwizzleA ? q0 ^ col : q0));
                a1[t] = *reinterpret_cast<const u32x4*>(ap + 16 * (kSwizzleA ? (q0 + 1) ^ col : q0 + 1));
            }
#pragma unroll
            for (int t = 0; t < MT; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a0[t]), b0, acc[t], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < MT; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a1[t]), b1, acc[t], 0, 0, 0);
        }
        __builtin_amdgcn_wave_barrier();
    };
    // The turn count is rounded up to even: an extra turn past the slice
    // is skipped by multiply. (Leaving the loop after an odd turn instead lets
    // the compiler sink the next turn's loads below the multiply.)
    const int nt = (c1 - c0 + G - 1) / G;
    u32x4 bv0[2], bv1[2];
    u32x4 ar0[kP], ar1[kP];
    load(bv0, ar0, c0);
    for (int i = 0; i < nt; i += 2) {
        stage(0, ar0);
        __syncthreads();
        load(bv1, ar1, c0 + G * (i + 1));
        __builtin_amdgcn_sched_barrier(0);
        multiply(0, bv0, c0 + G * i);
        stage(1, ar1);
        __syncthreads();
        load(bv0, ar0, c0 + G * (i + 2));
        __builtin_amdgcn_sched_barrier(0);
        multiply(1, bv1, c0 + G * (i + 1));
    }

    if (G > 1) {
        // Groups 1 .. G-1 hand their sums to group 0 through the A buffers
        // (free once every wave has passed this barrier), which adds them in
        // group order.
        __syncthreads();
        f32x4* red = reinterpret_cast<f32x4*>(&lds_a[0][0][0]);
        if (kg > 0) {
#pragma unroll
            for (int t = 0; t < MT; ++t) red[(((kg - 1) * W + wv) * MT + t) * kWave + lane] = acc[t];
        }
        __syncthreads();
        // SW keeps every wave to the epilogue's barriers.
        if (!SW && kg > 0) return;
        if (kg == 0) {
#pragma unroll
            for (int g = 1; g < G; ++g)
#pragma unroll
                for (int t = 0; t < MT; ++t) acc[t] += red[(((g - 1) * W + wv) * MT + t) * kWave + lane];
        }
    }
    if constexpr (SW) {
        // gate, up and SwiGLU (one K slice): the up waves of group 0 store
        // their rounded values, the gate waves of group 0 combine.
        __syncthreads();  // the group sums' reads of the A buffers are done
        uint16_t* xch = reinterpret_cast<uint16_t*>(&lds_a[0][0][0]);  // [W/2][MT][4][64]
        const int wp = wv % (W / 2);
        if (kg == 0 && upw && n < N) {
            const float sc = scale[n];
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) xch[((wp * MT + t) * 4 + e) * kWave + lane] = from_f32<f16>(acc[t][e] * sc);
        }
        __syncthreads();
        if (kg == 0 && !upw && n < N) {
            const float sc = scale[n];
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = 16 * t + 4 * grp + e;
                    if (m < M) {
                        const size_t o = static_cast<size_t>(m) * N + n;
                        const uint16_t gv = from_f32<f16>(acc[t][e] * sc);
                        const uint16_t uv = xch[((wp * MT + t) * 4 + e) * kWave + lane];
                        sw->gate[o] = gv;
                        sw->up[o] = uv;
                        sw->out[o] = from_f32<f16>(swiglu_f32(to_f32<f16>(gv), to_f32<f16>(uv)));
                    }
                }
        }
        return;
    }
    if (S == 1) {
        if (n < N) {
            const float sc = scale[n];
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = 16 * t + 4 * grp + e;
                    if (m < M) c[static_cast<size_t>(m) * N + n] = from_f32<f16>(acc[t][e] * sc);
                }
        }
        return;
    }
    if (n < N) {
        float* mine = part + static_cast<size_t>(sl) * Mall * N;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = 16 * t + 4 * grp + e;
                if (m < M) mine[static_cast<size_t>(m) * N + n] = acc[t][e];
            }
    }
}

template <int MT, int W, int G>
__global__ __launch_bounds__(G * W * kWave) void gemm_i8w_split_kernel(
    uint16_t* __restrict__ c, const uint16_t* __restrict__ a, const int8_t* __restrict__ b,
    const float* __restrict__ scale, float* __restrict__ part, int M, int N, int K, int S, int tiles, int cps,
    int TT) {
    gemm_i8w_split_block<MT, W, G>(c, a, b, scale, part, M, N, K, S, tiles, cps, TT, blockIdx.x);
}

// gate/up and SwiGLU on the split kernel (ng_gemm_int8_silu_mul from 3 rows):
// one K slice, blocks of 8 W row pairs.
template <int MT, int W, int G>
__global__ __launch_bounds__(G * W * kWave) void gemm_i8w_split_swiglu_kernel(SwigluArgs sa,
                                                                               const uint16_t* __restrict__ a,
                                                                               int M, int N, int K, int cps) {
    gemm_i8w_split_block<MT, W, G, true>(nullptr, a, nullptr, nullptr, nullptr, M, N, K, 1, 0, cps, 1, blockIdx.x,
                                         &sa);
}

// Products that share A on one split-kernel shape (ng_gemm_int8_shared_a):
// each product keeps its own slices of K and its own region of the
// partial-sum buffer, so its sums are those of its own launch.
template <int MT, int W, int G>
__global__ __launch_bounds__(G * W * kWave) void gemm_i8w_split_shared_kernel(SharedSet s, SplitSet sp,
                                                                               const uint16_t* __restrict__ a, int M,
                                                                               int K) {
    shared_dispatch(s, [&](uint16_t* c, const int8_t* b, const float* scale, int n, int blk, int p) {
        gemm_i8w_split_block<MT, W, G>(c, a, b, scale, pick4(p, sp.part[0], sp.part[1], sp.part[2], sp.part[3]), M,
                                       n, K, pick4(p, sp.S[0], sp.S[1], sp.S[2], sp.S[3]),
                                       pick4(p, sp.tiles[0], sp.tiles[1], sp.tiles[2], sp.tiles[3]),
                                       pick4(p, sp.cps[0], sp.cps[1], sp.cps[2], sp.cps[3]),
                                       pick4(p, sp.TT[0], sp.TT[1], sp.TT[2], sp.TT[3]), blk);
    });
}

// C[m, n] = fp16(scale[n] * sum over slices q = 0 .. S-1, in that order, of
// part[q][m][n]), S <= 8. Four outputs per thread when N % 4 == 0 (16-byte
// loads of the partial sums and scales, one 8-byte store), else one. Every
// slice is loaded before the first addition (slices past S reload slice 0),
// so the loads overlap: 1.3-1.5 us faster than a loop of dependent loads
// with 8 slices.
// The residual add after a product (ng_gemm_int8_add): out = fp16(C + res) on
// the rounded C, as cuda_add computes it. out may be C or res itself (each
// element is read and written by one thread, out last).
struct ResEpi {
    uint16_t* out;
    const uint16_t* res;
};

// Outputs i .. i + 3 (N % 4 == 0) and output t of the reduction, rounded.
__device__ __forceinline__ u32x2 reduce_slices4(const float* __restrict__ part, const float* __restrict__ scale,
                                                size_t mn, int N, int S, size_t i) {
    f32x4 pv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q)
        pv[q] = *reinterpret_cast<const f32x4*>(part + static_cast<size_t>(q < S ? q : 0) * mn + i);
    f32x4 v = pv[0];
#pragma unroll
    for (int q = 1; q < 8; ++q)
        if (q < S) v += pv[q];
    const f32x4 sc = *reinterpret_cast<const f32x4*>(scale + i % N);
    return u32x2{pack2<f16>(v[0] * sc[0], v[1] * sc[1]), pack2<f16>(v[2] * sc[2], v[3] * sc[3])};
}

__device__ __forceinline__ uint16_t reduce_slices1(const float* __restrict__ part, const float* __restrict__ scale,
                                                   size_t mn, int N, int S, size_t t) {
    float pv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) pv[q] = part[static_cast<size_t>(q < S ? q : 0) * mn + t];
    float v = pv[0];
#pragma unroll
    for (int q = 1; q < 8; ++q)
        if (q < S) v += pv[q];
    return from_f32<f16>(v * scale[t % N]);
}

template <bool VEC4, bool RES = false>
__device__ __forceinline__ void split_reduce_block(uint16_t* c, const float* __restrict__ part,
                                                   const float* __restrict__ scale, int M, int N, int S, int blk,
                                                   const ResEpi& ep = ResEpi{}) {
    const size_t mn = static_cast<size_t>(M) * N;
    const size_t t = static_cast<size_t>(blk) * 256 + threadIdx.x;
    if (VEC4) {
        const size_t i = 4 * t;
        if (i >= mn) return;
        const u32x2 out = reduce_slices4(part, scale, mn, N, S, i);
        if (RES) {
            const u32x2 rv = *reinterpret_cast<const u32x2*>(ep.res + i);
            *reinterpret_cast<u32x2*>(c + i) = out;
            u32x2 sum;
#pragma unroll
            for (int h = 0; h < 2; ++h)
                sum[h] = pack2<f16>(el_add<f16, 0>(out[h], rv[h]), el_add<f16, 1>(out[h], rv[h]));
            *reinterpret_cast<u32x2*>(ep.out + i) = sum;
        } else {
            *reinterpret_cast<u32x2*>(c + i) = out;
        }
    } else {
        if (t >= mn) return;
        const uint16_t cv = reduce_slices1(part, scale, mn, N, S, t);
        if (RES) {
            const float sum = to_f32<f16>(cv) + to_f32<f16>(ep.res[t]);
            c[t] = cv;
            ep.out[t] = from_f32<f16>(sum);
        } else {
            c[t] = cv;
        }
    }
}

template <bool VEC4, bool RES = false>
__global__ __launch_bounds__(256) void split_reduce_kernel(uint16_t* c, const float* __restrict__ part,
                                                           const float* __restrict__ scale, int M, int N, int S,
                                                           ResEpi ep = ResEpi{}) {
    split_reduce_block<VEC4, RES>(c, part, scale, M, N, S, blockIdx.x, ep);
}

// gate/up with several K slices and SwiGLU (ng_gemm_int8_silu_mul): each
// thread reduces its outputs of both products as split_reduce_block does,
// stores gate and up, then out = fp16(silu(gate) * up) (out may be gate or
// up itself: each element is written by one thread, out last).
template <bool VEC4>
__global__ __launch_bounds__(256) void split_reduce_swiglu_kernel(SwigluArgs sa, const float* __restrict__ pg,
                                                                  const float* __restrict__ pu, int M, int N,
                                                                  int S) {
    const size_t mn = static_cast<size_t>(M) * N;
    const size_t t = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (VEC4) {
        const size_t i = 4 * t;
        if (i >= mn) return;
        const u32x2 g = reduce_slices4(pg, sa.sg, mn, N, S, i);
        const u32x2 u = reduce_slices4(pu, sa.su, mn, N, S, i);
        u32x2 o;
#pragma unroll
        for (int h = 0; h < 2; ++h)
            o[h] = pack2<f16>(swiglu_f32(el_get<f16, 0>(g[h]), el_get<f16, 0>(u[h])),
                              swiglu_f32(el_get<f16, 1>(g[h]), el_get<f16, 1>(u[h])));
        *reinterpret_cast<u32x2*>(sa.gate + i) = g;
        *reinterpret_cast<u32x2*>(sa.up + i) = u;
        *reinterpret_cast<u32x2*>(sa.out + i) = o;
    } else {
        if (t >= mn) return;
        const uint16_t g = reduce_slices1(pg, sa.sg, mn, N, S, t);
        const uint16_t u = reduce_slices1(pu, sa.su, mn, N, S, t);
        sa.gate[t] = g;
        sa.up[t] = u;
        sa.out[t] = from_f32<f16>(swiglu_f32(to_f32<f16>(g), to_f32<f16>(u)));
    }
}

// The reductions of the products of gemm_i8w_split_shared_kernel in one
// launch (blocks partitioned by product as in SharedSet).
template <bool VEC4>
__global__ __launch_bounds__(256) void split_reduce_shared_kernel(SharedSet s, SplitSet sp, int M) {
    shared_dispatch(s, [&](uint16_t* c, const int8_t*, const float* scale, int n, int blk, int p) {
        split_reduce_block<VEC4>(c, pick4(p, sp.part[0], sp.part[1], sp.part[2], sp.part[3]), scale, M, n,
                                 pick4(p, sp.S[0], sp.S[1], sp.S[2], sp.S[3]), blk);
    });
}


// ---- prefill variant (M > 128) ----------------------------------------------
// Many rows of A: the product is bound by the matrix cores, not by reading
// the weights. A block computes a BM x BN tile of C (BM = 16 TM WM rows of A,
// BN = 16 TN WN rows of B) with WM x WN waves, each a TM x TN grid of 16x16
// MFMA tiles, over a slice of K in steps of 64:
//   * the A tile (fp16) and the B tile go through LDS; the B codes are
//     converted to exact fp16 integers once, on their way into LDS, so a code
//     is converted once per block that uses it and the matrix cores read fp16;
//   * two LDS buffers: the loads of step kt + 1 are issued before step kt is
//     multiplied, then stored into the other buffer; one barrier per step;
//   * rows of 64 k are 128 bytes; piece q (16 bytes) of row r sits at
//     q xor ((r / 2) mod 8), so that the 16 lanes of an MFMA operand read
//     (rows r0 .. r0 + 15, one piece) hit 16 different 16-byte slots of the
//     256 bytes the banks serve per clock;
//   * A and B are read through buffer resources based at the block's first
//     row: 32-bit offsets, and rows past M (or N) read zeros;
//   * tiles are handed out XCD by XCD: consecutive block ids go to different
//     XCDs, so block b takes tile (b mod 8) * (tiles / 8) + b / 8, and the
//     tiles of one XCD (and of its L2) are neighbours, grouped kPfGroupM rows
//     of tiles at a time so that they share rows of A and of B;
//   * with S > 1 the K steps are split into S slices (slice-major over the
//     tiles); each block stores its fp32 sums in `part` [S][M][N] and
//     split_reduce_kernel adds the slices in slice order.
// Sums in fp32 in MFMA order; scale[n] multiplies the sum, as on the
// streaming paths. Launch shapes, measured on MI355X with random data
// (q_proj 4096 x 4096 at M = 4096: 16 waves of 64 x 64 on a 256 x 256 tile,
// 127 us, against 162 us for 4 waves on 128 x 128 and 169 us for 4 waves of
// 128 x 128 on 256 x 256, whose fragment loads the compiler serialises
// behind each group of MFMAs): 256 x 256 with 16 waves and no K slices when
// that gives 192 tiles or more, otherwise 128 x 128 with 4 waves and enough
// K slices for about 512 blocks.
constexpr int kPfBK = 64;
constexpr int kPfGroupM = 8;
constexpr int kPfBlocks = 512;

__device__ __forceinline__ int pf_slot(int row, int q) { return row * 8 + (q ^ ((row >> 1) & 7)); }

template <int TM, int TN, int WM, int WN>
__device__ __forceinline__ void gemm_i8w_prefill_block(
    uint16_t* __restrict__ c, const uint16_t* __restrict__ a, const int8_t* __restrict__ b,
    const float* __restrict__ scale, float* __restrict__ part, int M, int N, int K, int tiles_m, int tiles_n,
    int S, int cps, int blk) {
    constexpr int kThreads = WM * WN * kWave;
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    constexpr int kAP = BM * 8 / kThreads;  // 16-byte pieces (8 k) of A per thread per step
    constexpr int kBP = BN * 4 / kThreads;  // 16-code pieces of B per thread per step
    static_assert(BM * 8 % kThreads == 0 && BN * 4 % kThreads == 0, "tile pieces must divide among the threads");
    static_assert((kThreads / 8) % 16 == 0 && (kThreads / 4) % 16 == 0, "row strides must keep the swizzle");
    __shared__ __align__(16) u32x4 lds_a[2][BM * 8];
    __shared__ __align__(16) u32x4 lds_b[2][BN * 8];

    const int ntiles = tiles_m * tiles_n;
    int t = blk;
    if ((ntiles * S) % 8 == 0) t = (t % 8) * (ntiles * S / 8) + t / 8;
    const int sl = t / ntiles;
    t -= sl * ntiles;
    const int per_group = kPfGroupM * tiles_n;
    const int grp0 = (t / per_group) * kPfGroupM;
    const int gm = min(kPfGroupM, tiles_m - grp0);
    const int tm = grp0 + (t % per_group) % gm;
    const int tn = (t % per_group) / gm;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int wm = wave / WN, wn = wave % WN;

    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a + static_cast<size_t>(m0) * K), 0,
        static_cast<int>(min(static_cast<long long>(M - m0) * K * 2, 0x7fffffffll)), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(b + static_cast<size_t>(n0) * K), 0,
        static_cast<int>(min(static_cast<long long>(N - n0) * K, 0x7fffffffll)), 0x00020000);
    // Thread tid loads A pieces (row tid / 8 + j kThreads / 8, piece tid % 8)
    // and B pieces (row tid / 4 + j kThreads / 4, codes 16 (tid % 4) ..).
    const int aq = tid & 7, bp = tid & 3;
    const uint32_t aoff0 = static_cast<uint32_t>((tid >> 3) * K * 2 + 16 * aq);
    const uint32_t boff0 = static_cast<uint32_t>((tid >> 2) * K + 16 * bp);
    const uint32_t astride = static_cast<uint32_t>((kThreads / 8) * K * 2);
    const uint32_t bstride = static_cast<uint32_t>((kThreads / 4) * K);
    const int aslot0 = pf_slot(tid >> 3, aq);
    const int bslot0 = pf_slot(tid >> 2, 2 * bp), bslot1 = pf_slot(tid >> 2, 2 * bp + 1);

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jn = 0; jn < TN; ++jn) acc[i][jn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int nk = (K + kPfBK - 1) / kPfBK;
    const int c0 = sl * cps, c1 = min(nk, c0 + cps);
    u32x4 ra[kAP], rb[kBP];
    // Loads of step kt. In a last step that runs past K (K % 64 != 0) the
    // pieces past K are zeroed in both operands, so that they add nothing (an
    // inf times a zero would be NaN). The step offset is part of the vector
    // offset, which the buffer's range check covers: a piece past K of the
    // last row of A or B lies past num_records and reads zeros without a
    // memory access (pieces past K of other rows read the next row, in
    // bounds, and are zeroed here).
    auto load = [&](int kt) {
        const int k0 = kt * kPfBK;
#pragma unroll
        for (int j = 0; j < kAP; ++j)
            ra[j] = __builtin_amdgcn_raw_buffer_load_b128(rsa, aoff0 + j * astride + static_cast<uint32_t>(2 * k0), 0, 0);
#pragma unroll
        for (int j = 0; j < kBP; ++j)
            rb[j] = __builtin_amdgcn_raw_buffer_load_b128(rsb, boff0 + j * bstride + static_cast<uint32_t>(k0), 0, 0);
        if (k0 + kPfBK > K) {
            if (k0 + 8 * aq >= K) {
#pragma unroll
                for (int j = 0; j < kAP; ++j) ra[j] = u32x4{0u, 0u, 0u, 0u};
            }
            if (k0 + 16 * bp >= K) {
#pragma unroll
                for (int j = 0; j < kBP; ++j) rb[j] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int j = 0; j < kAP; ++j) lds_a[buf][aslot0 + j * (kThreads / 8) * 8] = ra[j];
#pragma unroll
        for (int j = 0; j < kBP; ++j) {
            f16x8 lo, hi;
            codes16_to_operands(rb[j], lo, hi);
            lds_b[buf][bslot0 + j * (kThreads / 4) * 8] = __builtin_bit_cast(u32x4, lo);
            lds_b[buf][bslot1 + j * (kThreads / 4) * 8] = __builtin_bit_cast(u32x4, hi);
        }
    };
    const int ar0 = wm * TM * 16 + (lane & 15);
    const int br0 = wn * TN * 16 + (lane & 15);
    auto frags = [&](int buf, int s2, u32x4 (&af)[TM], u32x4 (&bf)[TN]) {
        const int q = 4 * s2 + (lane >> 4);
#pragma unroll
        for (int i = 0; i < TM; ++i) af[i] = lds_a[buf][pf_slot(ar0 + 16 * i, q)];
#pragma unroll
        for (int jn = 0; jn < TN; ++jn) bf[jn] = lds_b[buf][pf_slot(br0 + 16 * jn, q)];
    };
    auto mma = [&](const u32x4 (&af)[TM], const u32x4 (&bf)[TN]) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int jn = 0; jn < TN; ++jn)
                acc[i][jn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, af[i]),
                                                                    __builtin_bit_cast(f16x8, bf[jn]), acc[i][jn],
                                                                    0, 0, 0);
    };

    if (c0 < c1) {
        load(c0);
        stage(0);
        __syncthreads();
        for (int kt = c0; kt < c1; ++kt) {
            const int buf = (kt - c0) & 1;
            if (kt + 1 < c1) load(kt + 1);
            u32x4 af0[TM], bf0[TN], af1[TM], bf1[TN];
            frags(buf, 0, af0, bf0);
            frags(buf, 1, af1, bf1);
            mma(af0, bf0);
            mma(af1, bf1);
            if (kt + 1 < c1) stage(buf ^ 1);
            __syncthreads();
        }
    }

    const int mb = m0 + wm * TM * 16 + 4 * (lane >> 4);
#pragma unroll
    for (int jn = 0; jn < TN; ++jn) {
        const int n = n0 + wn * TN * 16 + 16 * jn + (lane & 15);
        if (n >= N) continue;
        if (S == 1) {
            const float sc = scale[n];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = mb + 16 * i + e;
                    if (m < M) c[static_cast<size_t>(m) * N + n] = from_f32<f16>(acc[i][jn][e] * sc);
                }
        } else {
            float* mine = part + static_cast<size_t>(sl) * M * N;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = mb + 16 * i + e;
                    if (m < M) mine[static_cast<size_t>(m) * N + n] = acc[i][jn][e];
                }
        }
    }
}

template <int TM, int TN, int WM, int WN>
__global__ __launch_bounds__(WM * WN * kWave, 1) void gemm_i8w_prefill_kernel(
    uint16_t* __restrict__ c, const uint16_t* __restrict__ a, const int8_t* __restrict__ b,
    const float* __restrict__ scale, float* __restrict__ part, int M, int N, int K, int tiles_m, int tiles_n,
    int S, int cps) {
    gemm_i8w_prefill_block<TM, TN, WM, WN>(c, a, b, scale, part, M, N, K, tiles_m, tiles_n, S, cps, blockIdx.x);
}

// Products that share A on one prefill tile shape (ng_gemm_int8_shared_a):
// each product keeps its own tiles, K slices and partial-sum region. In
// SplitSet, `tiles` holds the product's tiles along N and `TT` its tiles
// along M. A product's blocks keep their own launch's placement on the XCDs up
// to a rotation: the tiles that one launch gives to one XCD still share one.
template <int TM, int TN, int WM, int WN>
__global__ __launch_bounds__(WM * WN * kWave, 1) void gemm_i8w_prefill_shared_kernel(SharedSet s, SplitSet sp,
                                                                                     const uint16_t* __restrict__ a,
                                                                                     int M, int K) {
    shared_dispatch(s, [&](uint16_t* c, const int8_t* b, const float* scale, int n, int blk, int p) {
        gemm_i8w_prefill_block<TM, TN, WM, WN>(c, a, b, scale, pick4(p, sp.part[0], sp.part[1], sp.part[2], sp.part[3]),
                                               M, n, K, pick4(p, sp.TT[0], sp.TT[1], sp.TT[2], sp.TT[3]),
                                               pick4(p, sp.tiles[0], sp.tiles[1], sp.tiles[2], sp.tiles[3]),
                                               pick4(p, sp.S[0], sp.S[1], sp.S[2], sp.S[3]),
                                               pick4(p, sp.cps[0], sp.cps[1], sp.cps[2], sp.cps[3]), blk);
    });
}

// ---- hipBLASLt path ----------------------------------------------------------
constexpr size_t kLtWorkspace = size_t(32) << 20;

#define NG_LT_CHECK(call)                                                                      \
    do {                                                                                       \
        hipblasStatus_t ng_st_ = (call);                                                       \
        if (ng_st_ != HIPBLAS_STATUS_SUCCESS) {                                                \
            fprintf(stderr, "neurogrid-amd: %s:%d: hipBLASLt status %d\n", __FILE__, __LINE__, \
                    static_cast<int>(ng_st_));                                                 \
            return -1;                                                                         \
        }                                                                                      \
    } while (0)

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t lw = nullptr, lx = nullptr, ly = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t ws = 0;
};

// Buffers of one (device, stream) pair: the library workspace, the fp16 copy
// of the weights, and the split-K partial sums. Work on one
// stream is ordered, so reusing them from call to call on that stream is safe;
// another stream gets its own.
struct StreamBuffers {
    void* ws = nullptr;
    size_t ws_bytes = 0;
    void* deq = nullptr;
    size_t deq_bytes = 0;
    void* part = nullptr;
    size_t part_bytes = 0;
};

using PlanKey = std::tuple<int, int, int, int, bool, bool, int>;  // device, M, K, N, transpose_a, transpose_b, ldc

std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<PlanKey, Plan> g_plans;
std::set<PlanKey> g_lt_refused;   // shapes hipBLASLt has no algorithm for, or refused
std::map<std::pair<int, hipStream_t>, StreamBuffers> g_buffers;
// Buffers replaced by larger ones. A HIP graph that captured an earlier call
// still names the old buffer, so it is kept until gemm_release().
std::vector<void*> g_retired;

int capturing(hipStream_t s, bool* out) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    NG_HIP_CHECK(hipStreamIsCapturing(s, &st));
    *out = st != hipStreamCaptureStatusNone;
    return 0;
}

// Make *p hold at least `need` bytes. Growing while the stream is being
// captured is refused: allocation cannot be captured. The old buffer is
// retired, not freed, so that graphs captured before the growth stay valid;
// a new buffer is at least twice the old one, which bounds what is retired by
// the final size. Caller holds g_mu.
int grow(hipStream_t s, void** p, size_t* have, size_t need) {
    if (need <= *have) return 0;
    bool cap = false;
    if (capturing(s, &cap) != 0) return -1;
    NG_REQUIRE(!cap, "cuda_gemm: the stream is being captured and a buffer of %zu bytes must be allocated first; "
                     "make one call of this shape on the stream before capture", need);
    const size_t bytes = need > 2 * *have ? need : 2 * *have;
    void* fresh = nullptr;
    NG_HIP_CHECK(hipMalloc(&fresh, bytes));
    if (*p != nullptr) g_retired.push_back(*p);
    *p = fresh;
    *have = bytes;
    return 0;
}

// Plan for row-major C[M,N] = op(A) @ op(B), the rows of C ldc elements
// apart (ldc = N unless C is a column block of a wider matrix). hipBLASLt is
// column-major: the row-major matrices are their transposes, so it computes
// C^T = op(B)^T op(A)^T with B as its first operand (the same swap as
// matmul.cu:90-147).
int get_plan(int dev, int M, int K, int N, bool ta, bool tb, const Plan** out, int ldc = 0) {
    if (ldc == 0) ldc = N;
    const PlanKey key{dev, M, K, N, ta, tb, ldc};
    auto it = g_plans.find(key);
    if (it != g_plans.end()) {
        *out = &it->second;
        return 0;
    }
    auto h = g_handles.find(dev);
    if (h == g_handles.end()) {
        hipblasLtHandle_t handle = nullptr;
        NG_LT_CHECK(hipblasLtCreate(&handle));
        h = g_handles.emplace(dev, handle).first;
    }
    Plan p;
    NG_LT_CHECK(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
    const int32_t op_w = tb ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    const int32_t op_x = ta ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    NG_LT_CHECK(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_w, sizeof(op_w)));
    NG_LT_CHECK(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_x, sizeof(op_x)));
    if (tb) NG_LT_CHECK(hipblasLtMatrixLayoutCreate(&p.lw, HIP_R_16F, K, N, K));
    else NG_LT_CHECK(hipblasLtMatrixLayoutCreate(&p.lw, HIP_R_16F, N, K, N));
    if (ta) NG_LT_CHECK(hipblasLtMatrixLayoutCreate(&p.lx, HIP_R_16F, M, K, M));
    else NG_LT_CHECK(hipblasLtMatrixLayoutCreate(&p.lx, HIP_R_16F, K, M, K));
    NG_LT_CHECK(hipblasLtMatrixLayoutCreate(&p.ly, HIP_R_16F, N, M, ldc));
    hipblasLtMatmulPreference_t pref = nullptr;
    NG_LT_CHECK(hipblasLtMatmulPreferenceCreate(&pref));
    const uint64_t ws = kLtWorkspace;
    NG_LT_CHECK(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                                      sizeof(ws)));
    hipblasLtMatmulHeuristicResult_t res{};
    int found = 0;
    const hipblasStatus_t st =
        hipblasLtMatmulAlgoGetHeuristic(h->second, p.desc, p.lw, p.lx, p.ly, p.ly, pref, 1, &res, &found);
    hipblasLtMatmulPreferenceDestroy(pref);
    NG_LT_CHECK(st);
    NG_REQUIRE(found > 0, "cuda_gemm: hipBLASLt has no kernel for M=%d K=%d N=%d", M, K, N);
    p.algo = res.algo;
    p.ws = res.workspaceSize;
    *out = &g_plans.emplace(key, p).first->second;
    return 0;
}

// C = op(A) @ op(B) through hipBLASLt. With q != nullptr, B is first
// dequantized from the int8 codes q and their scales into this stream's fp16
// copy (matmul.cu:205-236), and the copy is the B of the product.
int gemm_lt(void* c, const void* a, const void* b, const void* q, const void* scale, int M, int K, int N, bool ta,
            bool tb) {
    int dev = 0;
    NG_HIP_CHECK(hipGetDevice(&dev));
    const hipStream_t s = stream();
    std::lock_guard<std::mutex> lock(g_mu);
    const Plan* p = nullptr;
    if (get_plan(dev, M, K, N, ta, tb, &p) != 0) return -1;
    StreamBuffers* sb = &g_buffers[{dev, s}];
    if (grow(s, &sb->ws, &sb->ws_bytes, p->ws) != 0) return -1;
    if (q != nullptr &&
        grow(s, &sb->deq, &sb->deq_bytes, static_cast<size_t>(K) * static_cast<size_t>(N) * 2) != 0)
        return -1;
    if (q != nullptr) {
        const int r = tb ? cuda_dequantize_weights(sb->deq, q, scale, N, K, 1)
                         : cuda_dequantize_weights(sb->deq, q, scale, K, N, 0);
        if (r != 0) return r;
        b = sb->deq;
    }
    const float alpha = 1.0f, beta = 0.0f;
    NG_LT_CHECK(hipblasLtMatmul(g_handles[dev], p->desc, &alpha, b, p->lw, a, p->lx, &beta, c, p->ly, c, p->ly,
                                &p->algo, sb->ws, p->ws, s));
    return 0;
}

// cuda_gemm_int8 from kLtMinM rows of A on, in the engine's layout (B int8
// [N, K], one scale per row): the reference's composition, dequantize then
// multiply (matmul.cu:205-236), through gemm_lt. It keeps a K x N fp16 copy
// of the weights in this (device, stream)'s buffer, grown to the largest
// weight seen (117 MB for a 14336 x 4096 projection), where the reference
// allocates and frees one per call. Measured on MI355X at M = 4096 for
// Mistral-7B's projections: 115 us for q/o against 161 us for the fused
// prefill kernel, 424 against 531 for gate/up, 367 against 467 for down, 48
// against 59 for k/v; at M = 512 the fused kernel is faster (37 against
// 42 us for q/o). Between 512 and 4096 rows the composition is not measured,
// so the fused kernel keeps those sizes. Returns 1 when hipBLASLt has no
// algorithm for the shape or refuses the call (remembered for the shape),
// having written nothing but the fp16 buffer: the caller then runs the fused
// prefill kernel.
constexpr int kLtMinM = 4096;

int gemm_lt_rows(void* c, const void* a, const void* q, const void* scale, int M, int K, int N) {
    int dev = 0;
    NG_HIP_CHECK(hipGetDevice(&dev));
    const hipStream_t s = stream();
    std::lock_guard<std::mutex> lock(g_mu);
    const PlanKey key{dev, M, K, N, false, true, N};
    if (g_lt_refused.count(key)) return 1;
    const Plan* p = nullptr;
    if (get_plan(dev, M, K, N, false, true, &p) != 0) {
        g_lt_refused.insert(key);
        return 1;
    }
    StreamBuffers* sb = &g_buffers[{dev, s}];
    if (grow(s, &sb->ws, &sb->ws_bytes, p->ws) != 0 ||
        grow(s, &sb->deq, &sb->deq_bytes, static_cast<size_t>(K) * static_cast<size_t>(N) * 2) != 0)
        return -1;
    const int r = cuda_dequantize_weights(sb->deq, q, scale, N, K, 1);
    if (r != 0) return r;
    const float alpha = 1.0f, beta = 0.0f;
    const hipblasStatus_t st = hipblasLtMatmul(g_handles[dev], p->desc, &alpha, sb->deq, p->lw, a, p->lx, &beta, c,
                                               p->ly, c, p->ly, &p->algo, sb->ws, p->ws, s);
    if (st != HIPBLAS_STATUS_SUCCESS) {
        // hipBLASLt's heuristic can name an algorithm that the call then
        // refuses (an internal error, status 6, at 4096 x 14336 x 512): the
        // shape goes to the fused kernel from now on, this call included.
        fprintf(stderr, "neurogrid-amd: hipBLASLt status %d at M=%d K=%d N=%d; using the fused kernel\n",
                static_cast<int>(st), M, K, N);
        g_lt_refused.insert(key);
        return 1;
    }
    return 0;
}

// The fp32 partial-sum buffer [S][M][N] of a split-K launch: `scratch` when
// the caller brings one (refused when too small), else this (device,
// stream)'s buffer, grown on demand with `lock` (g_mu) taken; the caller
// keeps the lock until both kernels are enqueued, so that calls from other
// host threads on the same stream cannot slip a launch between them.
int partial_buffer(hipStream_t s, int S, int M, int N, int K, float* scratch, size_t scratch_bytes,
                   std::unique_lock<std::mutex>& lock, float** out) {
    const size_t need = static_cast<size_t>(S) * M * N * sizeof(float);
    if (scratch != nullptr) {
        NG_REQUIRE(need <= scratch_bytes,
                   "ng_gemm_int8_noalloc: M=%d K=%d N=%d splits K into %d slices whose partial sums need %zu "
                   "bytes, more than the %zu-byte scratch; call cuda_gemm_int8 instead",
                   M, K, N, S, need, scratch_bytes);
        *out = scratch;
        return 0;
    }
    int dev = 0;
    NG_HIP_CHECK(hipGetDevice(&dev));
    lock.lock();
    StreamBuffers* sb = &g_buffers[{dev, s}];
    if (grow(s, &sb->part, &sb->part_bytes, need) != 0) return -1;
    *out = static_cast<float*>(sb->part);
    return 0;
}

// C = fp16(scale[n] * sum of the S slices of part), slices added in order.
int launch_reduce(hipStream_t s, uint16_t* c, const float* part, const float* scale, int M, int N, int S,
                  const ResEpi* ep = nullptr) {
    const size_t mn = static_cast<size_t>(M) * N;
    const dim3 b4(static_cast<unsigned>((mn / 4 + 255) / 256)), b1(static_cast<unsigned>((mn + 255) / 256));
    const bool vec4 = N % 4 == 0 && aligned16(scale) && aligned8(c) && (!ep || (aligned8(ep->out) && aligned8(ep->res)));
    if (ep) {
        if (vec4) split_reduce_kernel<true, true><<<b4, dim3(256), 0, s>>>(c, part, scale, M, N, S, *ep);
        else split_reduce_kernel<false, true><<<b1, dim3(256), 0, s>>>(c, part, scale, M, N, S, *ep);
    } else {
        if (vec4) split_reduce_kernel<true><<<b4, dim3(256), 0, s>>>(c, part, scale, M, N, S);
        else split_reduce_kernel<false><<<b1, dim3(256), 0, s>>>(c, part, scale, M, N, S);
    }
    NG_CHECK_LAUNCH("cuda_gemm_int8");
    return 0;
}

// Slices of K for a split launch of `tiles` tiles of B (and TT token tiles):
// enough for about 256 blocks (512 for K >= 8192; with G groups in the
// block, 192 blocks of twice the waves), at most 8, each of at least two
// turns, none empty; cps batches of 128 k per slice.
void split_slices(int tiles, int TT, int G, int K, int& S, int& cps) {
    const int nbatch = (K + kBatch - 1) / kBatch;
    const int target = G > 1 ? 192 : K >= 8192 ? 512 : 256;
    S = (target + tiles * TT - 1) / (tiles * TT);
    S = max(1, min(S, min(8, nbatch / (2 * G))));
    cps = (nbatch + S - 1) / S;
    S = (nbatch + cps - 1) / cps;
}

template <int MT, int W, int G>
int launch_split(uint16_t* c, const uint16_t* a, const int8_t* b, const float* scale, int M, int N, int K,
                 float* scratch, size_t scratch_bytes, int TT = 1, const ResEpi* ep = nullptr) {
    const int tiles = (N + 16 * W - 1) / (16 * W);
    int S = 0, cps = 0;
    split_slices(tiles, TT, G, K, S, cps);
    // With S > 1 the partial-sum buffer is this stream's: the lock is held
    // until both kernels are enqueued, so calls from other host threads on the
    // same stream cannot slip a launch between them.
    const hipStream_t s = stream();
    float* part = nullptr;
    std::unique_lock<std::mutex> lock(g_mu, std::defer_lock);
    if (S > 1 && partial_buffer(s, S, M, N, K, scratch, scratch_bytes, lock, &part) != 0) return -1;
    const int units = tiles * S;
    const int blocks = TT > 1 ? (units + 7) / 8 * 8 * TT : units;
    gemm_i8w_split_kernel<MT, W, G><<<dim3(static_cast<unsigned>(blocks)), dim3(G * W * kWave), 0, s>>>(
        c, a, b, scale, part, M, N, K, S, tiles, cps, TT);
    NG_CHECK_LAUNCH("cuda_gemm_int8");
    if (S > 1) return launch_reduce(s, c, part, scale, M, N, S, ep);
    return ep ? cuda_add(ep->out, c, ep->res, static_cast<size_t>(M) * N) : 0;
}

// The GEMV kernel gemm_i8w runs for a product on the weight-streaming path:
// 1 (one row of A, 8 rows of B per block), 2 (two rows of A, 8 of B), 3 (up
// to four rows of A, 4 of B), or 0 for the MFMA kernels. The GEMV kernel
// takes M <= 4 and K % 16 == 0, except M = 3, 4 with K or N of 8192 or more
// and K % 64 == 0, where the split kernel is faster.
int gemv_shape(int M, int K, int N) {
    const bool big = K >= 8192 || N >= 8192;
    if (M > 4 || K % 16 != 0 || (M >= 3 && big && K % kChunk == 0)) return 0;
    return M == 1 ? 1 : M == 2 ? 2 : 3;
}

// The split kernel's launch shape <MT, W, G> that gemm_i8w takes when the
// GEMV kernel does not, or kSmallM for the small-M MFMA kernel:
//   K >= 8192 (down): 8 waves per block;
//   N >= 12288 at smaller K (gate/up): 192 or more tiles of 64 rows fill the
//   GPU with one slice of K, split between two groups of 4 waves per block;
//   few rows of B (k/v: N = 1024 gives 16 tiles) and M > 32: blocks of 32
//   rows of A each (token tiles sharing B through one XCD's L2) instead of
//   one block for all of A: 7-16% faster at M = 64-128 (k/v: 9.0 vs 10.5 us
//   at M = 96); for larger N, and with 16-row token tiles, slower;
//   M <= 16 with K and N below 8192: the small-M MFMA kernel.
enum SplitConfig {
    kSmallM, kSplitTokenTiles, kSplit881, kSplit842, kSplit841, kSplit481, kSplit442, kSplit441, kSplit281,
    kSplit242, kSplit241, kSplit142, kSplit141
};
SplitConfig split_config(int M, int K, int N) {
    const bool big = K >= 8192 || N >= 8192;
    const bool deep = K >= 8192;
    const bool wide = !deep && N >= 12288;
    if (!deep && N <= 2048 && M > 32) return kSplitTokenTiles;
    if (M > 64) return deep ? kSplit881 : wide ? kSplit842 : kSplit841;
    if (M > 32) return deep ? kSplit481 : wide ? kSplit442 : kSplit441;
    if (M > 16) return deep ? kSplit281 : wide ? kSplit242 : kSplit241;
    if (big) return wide ? kSplit142 : kSplit141;
    return kSmallM;
}

// The launch shape gemm_i8w takes for a product on the weight-streaming
// path, for ng_gemm_int8_shared_a: the GEMV shapes 1-3 above, 4 for the
// small-M MFMA kernel, 10 + c for split shape c (10-22; the prefill kernel's
// shapes are kPathPrefill128 and kPathPrefill256).
int shared_path(int M, int K, int N) {
    const int gv = gemv_shape(M, K, N);
    if (gv != 0) return gv;
    const SplitConfig sc = split_config(M, K, N);
    return sc == kSmallM ? 4 : 10 + static_cast<int>(sc);
}

// Kernel and tile shape by M, K and N, from sweeps on MI355X over K x N in
// {4096 x 4096, 4096 x 1024, 4096 x 14336, 14336 x 4096} and M from 1 to 128:
// the GEMV kernel up to M = 4 (8 rows of B per block for M <= 2, 4 for M = 3,
// 4: 23-33% faster than the MFMA kernels at M = 1), the split kernel from
// M = 17 on and from M = 3 on with K or N of 8192 or more (at M = 4: 13.4 vs
// 14.8 us for gate/up, 13.7 vs 15.5 us for down), with token tiles of 32 rows
// of A for N <= 2048 from M = 33 on, otherwise the MFMA kernel that reads A
// from L2 directly.
// With ep, the residual add after the product follows: in the split-K
// reduction's epilogue where the launch has several K slices, else as
// cuda_add.
int gemm_i8w(void* c, const void* a, const void* b, const void* scale, int M, int K, int N,
             float* scratch = nullptr, size_t scratch_bytes = 0, const ResEpi* ep = nullptr) {
    auto* cp = static_cast<uint16_t*>(c);
    auto* ap = static_cast<const uint16_t*>(a);
    auto* bp = static_cast<const int8_t*>(b);
    auto* sp = static_cast<const float*>(scale);
    const auto then_add = [&](int r) {
        return r != 0 || !ep ? r : cuda_add(ep->out, c, ep->res, static_cast<size_t>(M) * N);
    };
    switch (gemv_shape(M, K, N)) {
        case 1: return then_add(launch_gemv<1, 8>(cp, ap, bp, sp, M, N, K));
        case 2: return then_add(launch_gemv<2, 8>(cp, ap, bp, sp, M, N, K));
        case 3: return then_add(launch_gemv<4, 4>(cp, ap, bp, sp, M, N, K));
        default: break;
    }
    switch (split_config(M, K, N)) {
        case kSplitTokenTiles: return launch_split<2, 4, 1>(cp, ap, bp, sp, M, N, K, scratch, scratch_bytes, (M + 31) / 32, ep);
        case kSplit881: return launch_split<8, 8, 1>(cp, ap, bp, sp, M, N, K, scratch, scratch_bytes, 1, ep);
        case kSplit842: return launch_split<8, 4, 2>(cp, ap, bp, sp, M, N, K, scratch, scratch_bytes, 1, ep);
        case kSplit841: return launch_split<8, 4, 1>(cp, ap, bp, sp, M, N, K, scratch, scratch_bytes, 1, ep);
        case kSplit481: return launch_split<4, 8, 1>(cp, ap, bp, sp, M, N, K, scratch, scratch_bytes, 1, ep);
        case kSplit442: return launch_split<4, 4, 2>(cp, ap, bp, sp, M, N, K, scratch, scratch_bytes, 1, ep);
        case kSplit441: return launch_split<4, 4, 1>(cp, ap, bp, sp, M, N, K, scratch, scratch_bytes, 1, ep);
        case kSplit281: return launch_split<2, 8, 1>(cp, ap, bp, sp, M, N, K, scratch, scratch_bytes, 1, ep);
        case kSplit242: return launch_split<2, 4, 2>(cp, ap, bp, sp, M, N, K, scratch, scratch_bytes, 1, ep);
        case kSplit241: return launch_split<2, 4, 1>(cp, ap, bp, sp, M, N, K, scratch, scratch_bytes, 1, ep);
        case kSplit142: return launch_split<1, 4, 2>(cp, ap, bp, sp, M, N, K, scratch, scratch_bytes, 1, ep);
        case kSplit141: return launch_split<1, 4, 1>(cp, ap, bp, sp, M, N, K, scratch, scratch_bytes, 1, ep);
        default: return then_add(launch_i8w<1, 1, 8, 4>(cp, ap, bp, sp, M, N, K));
    }
}

// The prefill kernel takes transpose_b, K % 16 == 0 and 16-byte aligned A and B.
bool use_prefill(const void* a, const void* b, int M, int K, int N, bool transpose_b) {
    return transpose_b && K % 16 == 0 && aligned16(a) && aligned16(b) &&
           static_cast<long long>(M) * K * 2 < (1ll << 31) && static_cast<long long>(N) * K < (1ll << 31);
}

// K slices of a prefill launch of `tiles` tiles of `area` outputs: for about
// kPfBlocks blocks, at most 8, each of 4 steps or more; none for 256 x 256
// tiles, which are only chosen when there are enough of them to fill the CUs.
void prefill_slices(int tiles, int area, int K, int& S, int& cps) {
    const int nk = (K + kPfBK - 1) / kPfBK;
    S = area >= 65536 ? 1 : max(1, min((kPfBlocks + tiles - 1) / tiles, min(8, nk / 4)));
    cps = (nk + S - 1) / S;
    S = (nk + cps - 1) / cps;
}

template <int TM, int TN, int WM, int WN>
int launch_prefill(uint16_t* c, const uint16_t* a, const int8_t* b, const float* scale, int M, int N, int K,
                   float* scratch, size_t scratch_bytes, const ResEpi* ep = nullptr) {
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const int tiles = tiles_m * tiles_n;
    int S = 0, cps = 0;
    prefill_slices(tiles, BM * BN, K, S, cps);
    const hipStream_t s = stream();
    float* part = nullptr;
    std::unique_lock<std::mutex> lock(g_mu, std::defer_lock);
    if (S > 1 && partial_buffer(s, S, M, N, K, scratch, scratch_bytes, lock, &part) != 0) return -1;
    gemm_i8w_prefill_kernel<TM, TN, WM, WN><<<dim3(static_cast<unsigned>(tiles * S)), dim3(WM * WN * kWave), 0, s>>>(
        c, a, b, scale, part, M, N, K, tiles_m, tiles_n, S, cps);
    NG_CHECK_LAUNCH("cuda_gemm_int8");
    if (S > 1) return launch_reduce(s, c, part, scale, M, N, S, ep);
    return ep ? cuda_add(ep->out, c, ep->res, static_cast<size_t>(M) * N) : 0;
}

// Tile shape by the number of tiles (see the prefill kernel): 256 x 256
// when that gives at least 192 tiles (three quarters of the CUs), otherwise
// 128 x 128 with K slices.
bool prefill_wide_tiles(int M, int N) {
    return static_cast<long long>((M + 255) / 256) * ((N + 255) / 256) >= 192;
}

// With ep, the residual add after the product follows, in the split-K
// reduction's epilogue where the launch slices K, else as cuda_add.
int gemm_prefill(void* c, const void* a, const void* b, const void* scale, int M, int K, int N,
                 float* scratch = nullptr, size_t scratch_bytes = 0, const ResEpi* ep = nullptr) {
    auto* cp = static_cast<uint16_t*>(c);
    auto* ap = static_cast<const uint16_t*>(a);
    auto* bp = static_cast<const int8_t*>(b);
    auto* sp = static_cast<const float*>(scale);
    if (prefill_wide_tiles(M, N))
        return launch_prefill<4, 4, 4, 4>(cp, ap, bp, sp, M, N, K, scratch, scratch_bytes, ep);
    return launch_prefill<4, 4, 2, 2>(cp, ap, bp, sp, M, N, K, scratch, scratch_bytes, ep);
}

// The weight-streaming path takes transpose_b, M <= kMaxFusedM, 16-byte aligned
// A and B, and K % 64 == 0 (K % 16 == 0 for M <= 4).
bool use_i8w(const void* a, const void* b, int M, int K, int N, bool transpose_b) {
    if (!transpose_b || M > kMaxFusedM || !aligned16(a) || !aligned16(b)) return false;
    return K % kChunk == 0 || (M <= 4 && K % 16 == 0);
}

// Device address of `scratch` on device `dev`, looked up with that device
// current on first use and kept per device (each device holds its own copy of
// the array at its own address).
constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch[kMaxDevices];

int scratch_ptr(int dev, float** out) {
    NG_REQUIRE(dev >= 0 && dev < kMaxDevices, "ng_gemm_int8_noalloc: device %d out of range", dev);
    float* p = g_scratch[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        void* addr = nullptr;
        NG_HIP_CHECK(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)));
        NG_REQUIRE(addr != nullptr, "ng_gemm_int8_noalloc: no device address for the scratch array");
        p = static_cast<float*>(addr);
        g_scratch[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return 0;
}

}  // namespace

int gemm_scratch_init(int dev) {
    float* p = nullptr;
    return scratch_ptr(dev, &p);
}

void gemm_release() {
    std::lock_guard<std::mutex> lock(g_mu);
    for (auto& kv : g_plans) {
        Plan& p = kv.second;
        hipblasLtMatrixLayoutDestroy(p.lw);
        hipblasLtMatrixLayoutDestroy(p.lx);
        hipblasLtMatrixLayoutDestroy(p.ly);
        hipblasLtMatmulDescDestroy(p.desc);
    }
    g_plans.clear();
    g_lt_refused.clear();
    for (auto& kv : g_buffers) {
        for (void* b : {kv.second.ws, kv.second.deq, kv.second.part})
            if (b != nullptr) (void)hipFree(b);
    }
    g_buffers.clear();
    for (void* b : g_retired) (void)hipFree(b);
    g_retired.clear();
    for (auto& kv : g_handles) hipblasLtDestroy(kv.second);
    g_handles.clear();
    // A device reset (cuda_shutdown) releases the module's device globals:
    // look the scratch array up again after the next initialisation.
    for (auto& p : g_scratch) p.store(nullptr, std::memory_order_release);
}

}  // namespace ng

using namespace ng;

extern "C" int cuda_gemm_fp16(void* c, const void* a, const void* b, int M, int K, int N, bool transpose_a,
                              bool transpose_b) {
    NG_REQUIRE(c && a && b, "cuda_gemm_fp16: null pointer");
    NG_REQUIRE(M > 0 && K > 0 && N > 0, "cuda_gemm_fp16: M=%d K=%d N=%d must be > 0", M, K, N);
    return gemm_lt(c, a, b, nullptr, nullptr, M, K, N, transpose_a, transpose_b);
}

extern "C" int cuda_gemm_int8(void* c, const void* a, const void* b, const void* scale, int M, int K, int N,
                              bool transpose_b) {
    NG_REQUIRE(c && a && b && scale, "cuda_gemm_int8: null pointer");
    NG_REQUIRE(M > 0 && K > 0 && N > 0, "cuda_gemm_int8: M=%d K=%d N=%d must be > 0", M, K, N);
    if (use_i8w(a, b, M, K, N, transpose_b)) return gemm_i8w(c, a, b, scale, M, K, N);
    if (use_prefill(a, b, M, K, N, transpose_b)) {
        if (M >= kLtMinM) {
            const int r = gemm_lt_rows(c, a, b, scale, M, K, N);
            if (r <= 0) return r;
        }
        return gemm_prefill(c, a, b, scale, M, K, N);
    }
    return gemm_lt(c, a, nullptr, b, scale, M, K, N, false, transpose_b);
}

// The fused paths of cuda_gemm_int8 with no allocation: their only buffer,
// the split-K partial sums, lives in this library's fixed `scratch` array of
// the current device. Same kernels, same launch shapes and so the same bits as
// cuda_gemm_int8 below kLtMinM rows of A; from kLtMinM rows on it keeps the
// fused prefill kernel, where cuda_gemm_int8 runs the dequantize + hipBLASLt
// composition. Every call on a device shares that device's
// array: calls that overlap on one GPU (other streams, other host threads)
// race on it. The split kernel writes every partial sum before the reduction
// reads it, so nothing needs clearing between calls.
extern "C" int ng_gemm_int8_noalloc(void* c, const void* a, const void* b, const void* scale, int M, int K, int N,
                                    bool transpose_b) {
    NG_REQUIRE(c && a && b && scale, "ng_gemm_int8_noalloc: null pointer");
    NG_REQUIRE(M > 0 && K > 0 && N > 0, "ng_gemm_int8_noalloc: M=%d K=%d N=%d must be > 0", M, K, N);
    const bool stream_path = use_i8w(a, b, M, K, N, transpose_b);
    NG_REQUIRE(stream_path || use_prefill(a, b, M, K, N, transpose_b),
               "ng_gemm_int8_noalloc: M=%d K=%d N=%d transpose_b=%d is outside the paths that run without "
               "allocating (transpose_b, K %% 16 == 0 (K %% 64 == 0 for 4 < M <= %d), 16-byte aligned A and B); "
               "call cuda_gemm_int8 instead", M, K, N, static_cast<int>(transpose_b), kMaxFusedM);
    int dev = 0;
    NG_HIP_CHECK(hipGetDevice(&dev));
    float* part = nullptr;
    if (scratch_ptr(dev, &part) != 0) return -1;
    if (stream_path) return gemm_i8w(c, a, b, scale, M, K, N, part, kNoAllocScratchBytes);
    return gemm_prefill(c, a, b, scale, M, K, N, part, kNoAllocScratchBytes);
}

// Per-product plan of a shared split-K launch: K slices, batches per slice,
// tiles along N and along M (the split kernel: token tiles), and blocks.
struct SharedPlan {
    int S[kMaxShared], cps[kMaxShared], tn[kMaxShared], tm[kMaxShared];
    long long blocks[kMaxShared];
};

// Products that share A on one split-K kernel shape: one launch of the kernel
// (`launch(set, sp, blocks, stream)`), then one of the reduction for the products with
// more than one slice of K, each product with its own slices and its own
// region of the stream's partial-sum buffer (the lock is held until both
// kernels are enqueued, as in launch_split).
// With sw (gate and up, both with several K slices, as count 2), the
// reduction is split_reduce_swiglu_kernel's; otherwise it returns 1 before
// launching anything.
template <typename L>
int run_shared_split(int count, void* const* c, const void* const* b, const void* const* scales, const int* n,
                     int M, int K, const SharedPlan& pl, L&& launch, const SwigluArgs* sw = nullptr) {
    if (sw && !(count == 2 && n[0] == n[1] && pl.S[0] > 1 && pl.S[1] == pl.S[0])) return 1;
    long long cols = 0;
    for (int i = 0; i < count; ++i)
        if (pl.S[i] > 1) cols += static_cast<long long>(pl.S[i]) * n[i];
    NG_REQUIRE(cols < (1ll << 31), "ng_gemm_int8_shared_a: too many rows of B");
    const hipStream_t st = stream();
    float* part = nullptr;
    std::unique_lock<std::mutex> lock(g_mu, std::defer_lock);
    if (cols > 0 && partial_buffer(st, 1, M, static_cast<int>(cols), K, nullptr, 0, lock, &part) != 0) return -1;
    SharedSet set{}, rset{};
    SplitSet sp{};
    long long blocks = 0, rblocks = 0, off = 0;
    bool vec4_all = true, vec4_any = false;
    for (int i = 0; i < kMaxShared; ++i) {
        const int j = i < count ? i : 0;  // unused slots repeat product 0 and are never selected
        set.c[i] = rset.c[i] = static_cast<uint16_t*>(c[j]);
        set.b[i] = rset.b[i] = static_cast<const int8_t*>(b[j]);
        set.scale[i] = rset.scale[i] = static_cast<const float*>(scales[j]);
        set.n[i] = rset.n[i] = n[j];
        sp.S[i] = pl.S[j];
        sp.tiles[i] = pl.tn[j];
        sp.cps[i] = pl.cps[j];
        sp.TT[i] = pl.tm[j];
        sp.part[i] = nullptr;
        set.first[i] = i < count ? static_cast<int>(blocks) : INT_MAX;
        rset.first[i] = i < count ? static_cast<int>(rblocks) : INT_MAX;
        if (i >= count) continue;
        blocks += pl.blocks[i];
        if (pl.S[i] > 1) {
            sp.part[i] = part + off;
            off += static_cast<long long>(pl.S[i]) * M * n[i];
            const bool v4 = n[i] % 4 == 0 && aligned16(scales[i]) && aligned8(c[i]);
            vec4_all = vec4_all && v4;
            vec4_any = vec4_any || v4;
            const long long mn = static_cast<long long>(M) * n[i];
            rblocks += v4 ? (mn / 4 + 255) / 256 : (mn + 255) / 256;
        }
        NG_REQUIRE(blocks < (1ll << 31) && rblocks < (1ll << 31), "ng_gemm_int8_shared_a: too many rows of B");
    }
    launch(set, sp, static_cast<unsigned>(blocks), st);
    NG_CHECK_LAUNCH("ng_gemm_int8_shared_a");
    if (sw) {
        const bool v4 = n[0] % 4 == 0 && aligned16(sw->sg) && aligned16(sw->su) && aligned8(sw->gate) &&
                        aligned8(sw->up) && aligned8(sw->out);
        const long long mn = static_cast<long long>(M) * n[0];
        const unsigned sb = static_cast<unsigned>(v4 ? (mn / 4 + 255) / 256 : (mn + 255) / 256);
        if (v4)
            split_reduce_swiglu_kernel<true><<<dim3(sb), dim3(256), 0, st>>>(*sw, sp.part[0], sp.part[1], M, n[0],
                                                                             pl.S[0]);
        else
            split_reduce_swiglu_kernel<false><<<dim3(sb), dim3(256), 0, st>>>(*sw, sp.part[0], sp.part[1], M, n[0],
                                                                              pl.S[0]);
        NG_CHECK_LAUNCH("ng_gemm_int8_silu_mul");
        return 0;
    }
    if (rblocks == 0) return 0;
    if (vec4_all || !vec4_any) {
        if (vec4_all)
            split_reduce_shared_kernel<true><<<dim3(static_cast<unsigned>(rblocks)), dim3(256), 0, st>>>(rset, sp, M);
        else
            split_reduce_shared_kernel<false><<<dim3(static_cast<unsigned>(rblocks)), dim3(256), 0, st>>>(rset, sp, M);
        NG_CHECK_LAUNCH("ng_gemm_int8_shared_a");
        return 0;
    }
    // Products whose reductions take different forms: one reduction each.
    for (int i = 0; i < count; ++i)
        if (pl.S[i] > 1 && launch_reduce(st, static_cast<uint16_t*>(c[i]), sp.part[i],
                                         static_cast<const float*>(scales[i]), M, n[i], pl.S[i]) != 0)
            return -1;
    return 0;
}

// The split kernel's shared form: slices and blocks as launch_split.
template <int MT, int W, int G>
int launch_split_shared(int count, void* const* c, const uint16_t* a, const void* const* b,
                        const void* const* scales, const int* n, int M, int K, int TT,
                        const SwigluArgs* sw = nullptr) {
    SharedPlan pl{};
    for (int i = 0; i < count; ++i) {
        pl.tn[i] = (n[i] + 16 * W - 1) / (16 * W);
        pl.tm[i] = TT;
        split_slices(pl.tn[i], TT, G, K, pl.S[i], pl.cps[i]);
        const long long units = static_cast<long long>(pl.tn[i]) * pl.S[i];
        pl.blocks[i] = TT > 1 ? (units + 7) / 8 * 8 * TT : units;
    }
    return run_shared_split(count, c, b, scales, n, M, K, pl,
                            [&](const SharedSet& set, const SplitSet& sp, unsigned blocks, hipStream_t st) {
                                gemm_i8w_split_shared_kernel<MT, W, G>
                                    <<<dim3(blocks), dim3(G * W * kWave), 0, st>>>(set, sp, a, M, K);
                            }, sw);
}

// The prefill kernel's shared form: tiles and slices as launch_prefill.
template <int TM, int TN, int WM, int WN>
int launch_prefill_shared(int count, void* const* c, const uint16_t* a, const void* const* b,
                          const void* const* scales, const int* n, int M, int K) {
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    SharedPlan pl{};
    for (int i = 0; i < count; ++i) {
        pl.tm[i] = (M + BM - 1) / BM;
        pl.tn[i] = (n[i] + BN - 1) / BN;
        prefill_slices(pl.tm[i] * pl.tn[i], BM * BN, K, pl.S[i], pl.cps[i]);
        pl.blocks[i] = static_cast<long long>(pl.tm[i]) * pl.tn[i] * pl.S[i];
    }
    return run_shared_split(count, c, b, scales, n, M, K, pl,
                            [&](const SharedSet& set, const SplitSet& sp, unsigned blocks, hipStream_t st) {
                                gemm_i8w_prefill_shared_kernel<TM, TN, WM, WN>
                                    <<<dim3(blocks), dim3(WM * WN * kWave), 0, st>>>(set, sp, a, M, K);
                            });
}

// Launch shapes of the fused prefill kernel for ng_gemm_int8_shared_a: 128 x 128
// tiles with K slices, or 256 x 256 tiles.
constexpr int kPathPrefill128 = 40, kPathPrefill256 = 41;

// One group of products that take the same launch shape `path` (see
// shared_path), in one launch of that kernel's shared form; shapes without a
// shared form, and groups of one, are one cuda_gemm_int8 call per product.
int shared_group(int path, int count, void* const* c, const void* a, const void* const* b,
                 const void* const* scales, const int* n, int M, int K) {
    const auto* ap = static_cast<const uint16_t*>(a);
    if (count > 1) {
        switch (path) {
            case 10 + kSplitTokenTiles:
                return launch_split_shared<2, 4, 1>(count, c, ap, b, scales, n, M, K, (M + 31) / 32);
            case 10 + kSplit141: return launch_split_shared<1, 4, 1>(count, c, ap, b, scales, n, M, K, 1);
            case 10 + kSplit241: return launch_split_shared<2, 4, 1>(count, c, ap, b, scales, n, M, K, 1);
            case 10 + kSplit441: return launch_split_shared<4, 4, 1>(count, c, ap, b, scales, n, M, K, 1);
            case 10 + kSplit841: return launch_split_shared<8, 4, 1>(count, c, ap, b, scales, n, M, K, 1);
            case 10 + kSplit142: return launch_split_shared<1, 4, 2>(count, c, ap, b, scales, n, M, K, 1);
            case 10 + kSplit242: return launch_split_shared<2, 4, 2>(count, c, ap, b, scales, n, M, K, 1);
            case 10 + kSplit442: return launch_split_shared<4, 4, 2>(count, c, ap, b, scales, n, M, K, 1);
            case 10 + kSplit842: return launch_split_shared<8, 4, 2>(count, c, ap, b, scales, n, M, K, 1);
            case kPathPrefill128: return launch_prefill_shared<4, 4, 2, 2>(count, c, ap, b, scales, n, M, K);
            case kPathPrefill256: return launch_prefill_shared<4, 4, 4, 4>(count, c, ap, b, scales, n, M, K);
            default: break;
        }
    }
    if (count == 1 || path <= 0 || path >= 10) {
        for (int i = 0; i < count; ++i) {
            const int r = cuda_gemm_int8(c[i], a, b[i], scales[i], M, K, n[i], true);
            if (r != 0) return r;
        }
        return 0;
    }
    const int R = path == 3 ? 4 : path == 4 ? 16 : 8;  // rows of B per block
    SharedSet set{};
    long long blocks = 0;
    for (int i = 0; i < kMaxShared; ++i) {
        const int j = i < count ? i : 0;  // unused slots repeat product 0 and are never selected
        set.c[i] = static_cast<uint16_t*>(c[j]);
        set.b[i] = static_cast<const int8_t*>(b[j]);
        set.scale[i] = static_cast<const float*>(scales[j]);
        set.n[i] = n[j];
        set.first[i] = i < count ? static_cast<int>(blocks) : INT_MAX;
        if (i < count) blocks += (n[i] + R - 1) / R;
        NG_REQUIRE(blocks < (1ll << 31), "ng_gemm_int8_shared_a: too many rows of B");
    }
    const int nb = static_cast<int>(blocks);
    switch (path) {
        case 1: return launch_gemv_shared<1, 8>(set, nb, ap, M, K);
        case 2: return launch_gemv_shared<2, 8>(set, nb, ap, M, K);
        case 3: return launch_gemv_shared<4, 4>(set, nb, ap, M, K);
        default:
            gemm_i8w_shared_kernel<1, 1, 8, 4><<<dim3(static_cast<unsigned>(nb)), dim3(8 * kWave), 0, stream()>>>(
                set, ap, M, K);
            NG_CHECK_LAUNCH("ng_gemm_int8_shared_a");
            return 0;
    }
}

// Products that share A (the engine's q/k/v and gate/up projections): they
// are grouped by the launch shape gemm_i8w would take for each, and each group
// runs in one launch of that kernel's shared form (plus one launch of the
// split kernel's reduction), each product's blocks exactly as its own launch
// would. Products outside the weight-streaming path are one cuda_gemm_int8
// call each. Either way the results are cuda_gemm_int8's, bit for bit.
extern "C" int ng_gemm_int8_shared_a(int count, void* const* c, const void* a, const void* const* b,
                                     const void* const* scales, const int* n, int M, int K) {
    NG_REQUIRE(c && a && b && scales && n, "ng_gemm_int8_shared_a: null pointer");
    NG_REQUIRE(count >= 1 && count <= kMaxShared, "ng_gemm_int8_shared_a: count=%d must be in [1, %d]", count,
               kMaxShared);
    NG_REQUIRE(M > 0 && K > 0, "ng_gemm_int8_shared_a: M=%d K=%d must be > 0", M, K);
    int path[kMaxShared];
    for (int i = 0; i < count; ++i) {
        NG_REQUIRE(c[i] && b[i] && scales[i], "ng_gemm_int8_shared_a: null pointer in product %d", i);
        NG_REQUIRE(n[i] > 0, "ng_gemm_int8_shared_a: n[%d]=%d must be > 0", i, n[i]);
        // cuda_gemm_int8's fused prefill kernel runs below kLtMinM rows of A
        path[i] = use_i8w(a, b[i], M, K, n[i], true) ? shared_path(M, K, n[i])
                  : M < kLtMinM && use_prefill(a, b[i], M, K, n[i], true)
                      ? (prefill_wide_tiles(M, n[i]) ? kPathPrefill256 : kPathPrefill128)
                      : 0;
    }
    bool done[kMaxShared] = {};
    for (int i = 0; i < count; ++i) {
        if (done[i]) continue;
        void* gc[kMaxShared];
        const void* gb[kMaxShared];
        const void* gs[kMaxShared];
        int gn[kMaxShared], g = 0;
        for (int j = i; j < count; ++j) {
            if (done[j] || path[j] != path[i] || (path[i] <= 0 && j != i)) continue;
            gc[g] = c[j];
            gb[g] = b[j];
            gs[g] = scales[j];
            gn[g] = n[j];
            ++g;
            done[j] = true;
        }
        const int r = shared_group(path[i], g, gc, a, gb, gs, gn, M, K);
        if (r != 0) return r;
    }
    return 0;
}

// [p, p + pn) and [q, q + qn) share a byte.
static bool overlaps(const void* p, size_t pn, const void* q, size_t qn) {
    const auto a = reinterpret_cast<uintptr_t>(p), b = reinterpret_cast<uintptr_t>(q);
    return a < b + qn && b < a + pn;
}

// RMSNorm (ADD: residual add + RMSNorm) of A, then the products that share
// the normalised A: one launch of gemv_i8w_norm_shared_kernel when every
// product takes the same GEMV shape of one or two rows, K <= 8192, the launch
// has at most kNormSharedMaxBlocks blocks and no output overlaps an input (the kernel's
// blocks read the inputs while the first one stores); otherwise the norm
// entry point followed by ng_gemm_int8_shared_a.
// The same bits either way. With rs, RoPE (ng_rope_qk_with_theta, style 0)
// follows on products 0 and 1 in place; the fused launch then also needs D a
// multiple of 8 (four rotation pairs per block of 8 rows of B), the three
// outputs apart from each other and the positions apart from every output.
struct RopeSpec {
    const int* pos;
    int nq, nkv, D;
    float theta;
};

template <bool ADD>
static int norm_shared(const char* name, int count, void* normed, void* res_out, void* const* c, const void* x,
                       const void* res, const void* w, float eps, const void* const* b, const void* const* scales,
                       const int* n, int M, int K, const RopeSpec* rs = nullptr) {
    NG_REQUIRE(normed && x && w && c && b && scales && n && (!ADD || (res && res_out)), "%s: null pointer", name);
    NG_REQUIRE(count >= 1 && count <= kMaxShared, "%s: count=%d must be in [1, %d]", name, count, kMaxShared);
    NG_REQUIRE(M > 0 && K > 0, "%s: M=%d K=%d must be > 0", name, M, K);
    const size_t rows = static_cast<size_t>(M) * K * 2;
    int path = -1;
    const size_t wb = static_cast<size_t>(K) * 2;
    // Nothing the blocks read may share a byte with what the first block
    // writes (normed, residual_out) or what any block writes (c).
    const auto clear_of_writes = [&](const void* p, size_t pn) {
        return !overlaps(p, pn, normed, rows) && (!ADD || !overlaps(p, pn, res_out, rows));
    };
    bool apart = clear_of_writes(x, rows) && clear_of_writes(w, wb) &&
                 (!ADD || (clear_of_writes(res, rows) && !overlaps(res_out, rows, normed, rows)));
    for (int i = 0; i < count; ++i) {
        NG_REQUIRE(c[i] && b[i] && scales[i], "%s: null pointer in product %d", name, i);
        NG_REQUIRE(n[i] > 0, "%s: n[%d]=%d must be > 0", name, i, n[i]);
        const int pi = use_i8w(normed, b[i], M, K, n[i], true) ? gemv_shape(M, K, n[i]) : 0;
        path = (path == -1 || path == pi) ? pi : 0;
        const size_t cb = static_cast<size_t>(M) * n[i] * 2;
        apart = apart && clear_of_writes(b[i], static_cast<size_t>(n[i]) * K) &&
                clear_of_writes(scales[i], static_cast<size_t>(n[i]) * 4) && clear_of_writes(c[i], cb) &&
                !overlaps(c[i], cb, x, rows) && !overlaps(c[i], cb, w, wb) && (!ADD || !overlaps(c[i], cb, res, rows));
    }
    if (rs) {
        const size_t pb = static_cast<size_t>(M) * 4;
        apart = apart && !overlaps(rs->pos, pb, normed, rows) && (!ADD || !overlaps(rs->pos, pb, res_out, rows));
        for (int i = 0; i < count; ++i) {
            const size_t cb = static_cast<size_t>(M) * n[i] * 2;
            apart = apart && !overlaps(rs->pos, pb, c[i], cb);
            for (int j = i + 1; j < count; ++j) apart = apart && !overlaps(c[i], cb, c[j], static_cast<size_t>(M) * n[j] * 2);
        }
    }
    // GEMV blocks of the fused launch (rows of B per block as the GEMV kernel's).
    const int R = 8;
    long long blocks = 0;
    for (int i = 0; i < count; ++i) blocks += (n[i] + R - 1) / R;
    const bool fused = (path == 1 || path == 2) && apart && K <= kNormSharedMaxK && blocks <= kNormSharedMaxBlocks &&
                       aligned16(x) && aligned16(w) && aligned16(normed) &&
                       (!ADD || (aligned16(res) && aligned16(res_out))) &&
                       (!rs || (rs->D % 8 == 0 && rs->D <= 2 * kRopeEpiMaxHalf));
    if (!fused) {
        int r = ADD ? cuda_add_rmsnorm(normed, res_out, x, res, w, M, K, eps) : cuda_rmsnorm(normed, x, w, M, K, eps);
        if (r == 0) r = ng_gemm_int8_shared_a(count, c, normed, b, scales, n, M, K);
        if (r == 0 && rs)
            r = ng_rope_qk_with_theta(c[0], c[0], c[1], c[1], rs->pos, 1, M, rs->nq, rs->nkv, rs->D, 0, rs->theta);
        return r;
    }
    SharedSet set{};
    int first = 0;
    for (int i = 0; i < kMaxShared; ++i) {
        const int j = i < count ? i : 0;  // unused slots repeat product 0 and are never selected
        set.c[i] = static_cast<uint16_t*>(c[j]);
        set.b[i] = static_cast<const int8_t*>(b[j]);
        set.scale[i] = static_cast<const float*>(scales[j]);
        set.n[i] = n[j];
        set.first[i] = i < count ? first : INT_MAX;
        if (i < count) first += (n[i] + R - 1) / R;
    }
    const NormArgs na{static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(res), static_cast<const uint16_t*>(w),
                      static_cast<uint16_t*>(normed), static_cast<uint16_t*>(res_out), eps};
    if constexpr (!ADD) {
        if (rs) {
            RopeEpi re{};
            re.pos = rs->pos;
            re.D = rs->D;
            re.half = rs->D / 2;
            re.bph = rs->D / 8;
            fill_inv_freq(rs->theta, rs->D, re.inv_freq);
            const dim3 grid(static_cast<unsigned>(first)), block(kGvWaves * kWave);
            const bool one = K <= kGvWaves * kGvSeg;
            if (path == 1) {
                if (one) gemv_i8w_norm_rope_shared_kernel<1, 1><<<grid, block, 0, stream()>>>(set, na, re, M, K);
                else gemv_i8w_norm_rope_shared_kernel<1, 2><<<grid, block, 0, stream()>>>(set, na, re, M, K);
            } else {
                if (one) gemv_i8w_norm_rope_shared_kernel<2, 1><<<grid, block, 0, stream()>>>(set, na, re, M, K);
                else gemv_i8w_norm_rope_shared_kernel<2, 2><<<grid, block, 0, stream()>>>(set, na, re, M, K);
            }
            NG_CHECK_LAUNCH(name);
            return 0;
        }
    }
    if (path == 1) return launch_gemv_norm_shared<1, 8, ADD>(set, first, na, M, K);
    return launch_gemv_norm_shared<2, 8, ADD>(set, first, na, M, K);
}

extern "C" int ng_rmsnorm_gemm_int8_shared_a(int count, void* normed, void* const* c, const void* x,
                                             const void* norm_weight, float eps, const void* const* b,
                                             const void* const* scales, const int* n, int M, int K) {
    return norm_shared<false>("ng_rmsnorm_gemm_int8_shared_a", count, normed, nullptr, c, x, nullptr, norm_weight, eps,
                              b, scales, n, M, K);
}

extern "C" int ng_add_rmsnorm_gemm_int8_shared_a(int count, void* normed, void* residual_out, void* const* c,
                                                 const void* x, const void* residual_in, const void* norm_weight,
                                                 float eps, const void* const* b, const void* const* scales,
                                                 const int* n, int M, int K) {
    return norm_shared<true>("ng_add_rmsnorm_gemm_int8_shared_a", count, normed, residual_out, c, x, residual_in,
                             norm_weight, eps, b, scales, n, M, K);
}

extern "C" int ng_rmsnorm_qkv_rope_int8(void* normed, void* q, void* k, void* v, const void* x,
                                        const void* norm_weight, float eps, const void* const* b,
                                        const void* const* scales, const int* positions, int M, int hidden,
                                        int num_q_heads, int num_kv_heads, int head_dim, float rope_theta) {
    const char* name = "ng_rmsnorm_qkv_rope_int8";
    NG_REQUIRE(q && k && v && positions && b && scales, "%s: null pointer", name);
    NG_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0 && head_dim <= 256,
               "%s: num_q_heads=%d num_kv_heads=%d head_dim=%d (even, at most 256)", name, num_q_heads, num_kv_heads,
               head_dim);
    NG_REQUIRE(static_cast<long long>(num_q_heads) * head_dim < (1ll << 31) &&
                   static_cast<long long>(num_kv_heads) * head_dim < (1ll << 31),
               "%s: too many rows of B", name);
    void* c[3] = {q, k, v};
    const int n[3] = {num_q_heads * head_dim, num_kv_heads * head_dim, num_kv_heads * head_dim};
    const RopeSpec rs{positions, num_q_heads, num_kv_heads, head_dim, rope_theta};
    return norm_shared<false>(name, 3, normed, nullptr, c, x, nullptr, norm_weight, eps, b, scales, n, M, hidden, &rs);
}

// The split kernel's SwiGLU form: the launch shape <MT, W, G> that
// split_config gives each of gate and up, when it takes one K slice (the
// wide two-group shapes); 1 when it does not, so that the caller runs the
// two calls.
template <int MT, int W, int G>
int launch_split_swiglu(const SwigluArgs& sa, const uint16_t* a, int M, int N, int K) {
    const int tn = (N + 16 * W - 1) / (16 * W);  // tiles of one product's own launch
    int S = 0, cps = 0;
    split_slices(tn, 1, G, K, S, cps);
    if (S != 1) return 1;
    const unsigned blocks = static_cast<unsigned>((N + 8 * W - 1) / (8 * W));
    gemm_i8w_split_swiglu_kernel<MT, W, G><<<dim3(blocks), dim3(G * W * kWave), 0, stream()>>>(sa, a, M, N, K, cps);
    NG_CHECK_LAUNCH("ng_gemm_int8_silu_mul");
    return 0;
}

// gate/up with several K slices on a one-group split shape: the shared launch
// (partial sums only) and split_reduce_swiglu_kernel; 1 for other shapes.
static int swiglu_sliced(const SwigluArgs& sa, const uint16_t* a, int M, int K, int N) {
    void* c[2] = {sa.gate, sa.up};
    const void* b[2] = {sa.bg, sa.bu};
    const void* sc[2] = {sa.sg, sa.su};
    const int n[2] = {N, N};
    switch (shared_path(M, K, N)) {
        case 10 + kSplit141: return launch_split_shared<1, 4, 1>(2, c, a, b, sc, n, M, K, 1, &sa);
        case 10 + kSplit241: return launch_split_shared<2, 4, 1>(2, c, a, b, sc, n, M, K, 1, &sa);
        case 10 + kSplit441: return launch_split_shared<4, 4, 1>(2, c, a, b, sc, n, M, K, 1, &sa);
        case 10 + kSplit841: return launch_split_shared<8, 4, 1>(2, c, a, b, sc, n, M, K, 1, &sa);
        default: return 1;
    }
}

static int swiglu_split(const SwigluArgs& sa, const uint16_t* a, int M, int K, int N) {
    switch (split_config(M, K, N)) {
        case kSplit842: return launch_split_swiglu<8, 4, 2>(sa, a, M, N, K);
        case kSplit442: return launch_split_swiglu<4, 4, 2>(sa, a, M, N, K);
        case kSplit242: return launch_split_swiglu<2, 4, 2>(sa, a, M, N, K);
        case kSplit142: return launch_split_swiglu<1, 4, 2>(sa, a, M, N, K);
        default: return 1;
    }
}

// gate/up (cuda_gemm_int8 on one A, as ng_gemm_int8_shared_a) and SwiGLU
// (cuda_silu_mul), when no output overlaps an input or another output (out
// may be gate or up exactly): one launch of gemv_i8w_swiglu_kernel when both
// products take the GEMV kernel, one of gemm_i8w_split_swiglu_kernel when
// they take the split kernel with one K slice, the shared split launch and
// split_reduce_swiglu_kernel when they take a one-group split shape with
// several K slices; otherwise the two calls. The same bits either way.
extern "C" int ng_gemm_int8_silu_mul(void* out, void* gate, void* up, const void* a, const void* b_gate,
                                     const void* scale_gate, const void* b_up, const void* scale_up, int M, int K,
                                     int N) {
    NG_REQUIRE(out && gate && up && a && b_gate && scale_gate && b_up && scale_up, "ng_gemm_int8_silu_mul: null pointer");
    NG_REQUIRE(M > 0 && K > 0 && N > 0, "ng_gemm_int8_silu_mul: M=%d K=%d N=%d must be > 0", M, K, N);
    const size_t cb = static_cast<size_t>(M) * N * 2, ab = static_cast<size_t>(M) * K * 2;
    const size_t bb = static_cast<size_t>(N) * K, sb = static_cast<size_t>(N) * 4;
    const int path = use_i8w(a, b_gate, M, K, N, true) && use_i8w(a, b_up, M, K, N, true) ? gemv_shape(M, K, N) : 0;
    bool apart = !overlaps(gate, cb, up, cb) && (out == gate || out == up || (!overlaps(out, cb, gate, cb) &&
                                                                              !overlaps(out, cb, up, cb)));
    for (const void* o : {out, gate, up})
        apart = apart && !overlaps(o, cb, a, ab) && !overlaps(o, cb, b_gate, bb) && !overlaps(o, cb, b_up, bb) &&
                !overlaps(o, cb, scale_gate, sb) && !overlaps(o, cb, scale_up, sb);
    const SwigluArgs sa{static_cast<uint16_t*>(out), static_cast<uint16_t*>(gate), static_cast<uint16_t*>(up),
                        static_cast<const int8_t*>(b_gate), static_cast<const int8_t*>(b_up),
                        static_cast<const float*>(scale_gate), static_cast<const float*>(scale_up)};
    if (path < 1 && apart && use_i8w(a, b_gate, M, K, N, true) && use_i8w(a, b_up, M, K, N, true)) {
        int r = swiglu_split(sa, static_cast<const uint16_t*>(a), M, K, N);
        if (r == 1) r = swiglu_sliced(sa, static_cast<const uint16_t*>(a), M, K, N);
        if (r <= 0) return r;
    }
    if (path < 1 || !apart) {
        void* c[2] = {gate, up};
        const void* b[2] = {b_gate, b_up};
        const void* sc[2] = {scale_gate, scale_up};
        const int n[2] = {N, N};
        const int r = ng_gemm_int8_shared_a(2, c, a, b, sc, n, M, K);
        if (r != 0) return r;
        return cuda_silu_mul(out, gate, up, static_cast<size_t>(M) * N);
    }
    const auto ap = static_cast<const uint16_t*>(a);
    const dim3 block(kGvWaves * kWave);
    if (path == 3) {
        gemv_i8w_swiglu_kernel<4, 4><<<dim3(static_cast<unsigned>((N + 3) / 4)), block, 0, stream()>>>(sa, ap, M, N, K);
    } else if (path == 2) {
        gemv_i8w_swiglu_kernel<2, 8><<<dim3(static_cast<unsigned>((N + 7) / 8)), block, 0, stream()>>>(sa, ap, M, N, K);
    } else {
        gemv_i8w_swiglu_kernel<1, 8><<<dim3(static_cast<unsigned>((N + 7) / 8)), block, 0, stream()>>>(sa, ap, M, N, K);
    }
    NG_CHECK_LAUNCH("ng_gemm_int8_silu_mul");
    return 0;
}

// A product (cuda_gemm_int8 with transpose_b) and the residual add after it
// (cuda_add(out, c, residual)): when no output overlaps an input or the other
// output (out may be c or the residual exactly), one launch of
// gemv_i8w_add_kernel on the GEMV kernel's shapes, and on cuda_gemm_int8's
// other fused paths (the weight-streaming kernels up to 128 rows, the prefill
// kernel below kLtMinM) the add in the split-K reduction (after the product as
// cuda_add where the launch has one K slice); otherwise the two calls. The
// same bits either way.
extern "C" int ng_gemm_int8_add(void* out, void* c, const void* a, const void* b, const void* scale,
                                const void* residual, int M, int K, int N) {
    NG_REQUIRE(out && c && a && b && scale && residual, "ng_gemm_int8_add: null pointer");
    NG_REQUIRE(M > 0 && K > 0 && N > 0, "ng_gemm_int8_add: M=%d K=%d N=%d must be > 0", M, K, N);
    const size_t cb = static_cast<size_t>(M) * N * 2, ab = static_cast<size_t>(M) * K * 2;
    const size_t bb = static_cast<size_t>(N) * K, sb = static_cast<size_t>(N) * 4;
    const int path = use_i8w(a, b, M, K, N, true) ? gemv_shape(M, K, N) : 0;
    bool apart = !overlaps(c, cb, residual, cb) &&
                 (out == c || out == residual || (!overlaps(out, cb, c, cb) && !overlaps(out, cb, residual, cb)));
    for (const void* o : {out, c})
        apart = apart && !overlaps(o, cb, a, ab) && !overlaps(o, cb, b, bb) && !overlaps(o, cb, scale, sb);
    if (path < 1 || !apart) {
        // cuda_gemm_int8's own fused paths (the weight-streaming kernels up to
        // 128 rows of A, the prefill kernel below kLtMinM): the add in the
        // split-K reduction where the launch has one.
        const ResEpi ep{static_cast<uint16_t*>(out), static_cast<const uint16_t*>(residual)};
        if (apart && use_i8w(a, b, M, K, N, true)) return gemm_i8w(c, a, b, scale, M, K, N, nullptr, 0, &ep);
        if (apart && M < kLtMinM && use_prefill(a, b, M, K, N, true))
            return gemm_prefill(c, a, b, scale, M, K, N, nullptr, 0, &ep);
        const int r = cuda_gemm_int8(c, a, b, scale, M, K, N, true);
        if (r != 0) return r;
        return cuda_add(out, c, residual, static_cast<size_t>(M) * N);
    }
    const auto o16 = static_cast<uint16_t*>(out);
    const auto c16 = static_cast<uint16_t*>(c);
    const auto r16 = static_cast<const uint16_t*>(residual);
    const auto ap = static_cast<const uint16_t*>(a);
    const auto bp = static_cast<const int8_t*>(b);
    const auto sp = static_cast<const float*>(scale);
    const dim3 block(kGvWaves * kWave);
    if (path == 3) {
        gemv_i8w_add_kernel<4, 4><<<dim3(static_cast<unsigned>((N + 3) / 4)), block, 0, stream()>>>(
            o16, c16, r16, ap, bp, sp, M, N, K);
    } else if (path == 2) {
        gemv_i8w_add_kernel<2, 8><<<dim3(static_cast<unsigned>((N + 7) / 8)), block, 0, stream()>>>(
            o16, c16, r16, ap, bp, sp, M, N, K);
    } else {
        gemv_i8w_add_kernel<1, 8><<<dim3(static_cast<unsigned>((N + 7) / 8)), block, 0, stream()>>>(
            o16, c16, r16, ap, bp, sp, M, N, K);
    }
    NG_CHECK_LAUNCH("ng_gemm_int8_add");
    return 0;
}
