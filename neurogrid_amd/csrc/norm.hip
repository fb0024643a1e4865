// norm.hip - row kernels: RMSNorm, residual-add + RMSNorm, fused RMSNorm +
// per-token int8 quantisation, and per-row int8 absmax quantisation.
//
// Semantics (one row of H elements; fp32 arithmetic, IEEE division/sqrt):
//   s_i  = x_i                       (plain)   or  RN_f32(x_i + res_i)  (ADD)
//   ro_i = RN_T(s_i)                 residual_output (ADD only)
//   ss   = RN_f32(exact sum s_i^2)   see ng_exact.hpp
//   r    = 1 / sqrt(ss / H + eps)
//   y_i  = RN_T((o_i * r) * w_i),    o_i = x_i (plain) or ro_i (ADD)
// The reference computes the same quantities with an fp32 tree sum
// (gpu/cuda/kernels.cu:58-95 and 196-235; bf16_utils.cu:57-93).
// Quantisation of a row v (v = y for the fused kernels, v = x otherwise):
//   m = max|v_i| over the non-NaN v_i, scale = m / 127 (1 if 0),
//   q_i = fmaxf(-127, fminf(127, rint(v_i / scale)))
// (reference: quantize.cu:274-316, with half-to-even rounding), where
// v_i / scale is the IEEE quotient, obtained without a division (qcode8).
// As in the reference, a NaN element is skipped by the maximum and gets the
// code +127; a row holding one takes the division path (qcode8_div).
//
// Every element-wise step is a single fp32 rounding; for fp16 rows the steps
// read their fp16 operands directly (v_fma_mix_f32, see el_mul / el_add), so
// the kernels spend about 6 VALU operations per element (13 with int8 codes)
// and stay under the HBM time. The sum of squares runs in fp64 (exact
// squares, any order) and is resolved to RN_f32 against a rigorous error
// bound, with an exact fallback (ng_exact.hpp).
//
// Layout: one workgroup per row, the row held in registers. Lane l of a
// workgroup of nthr threads owns the 16-byte vectors l, l + nthr, ...; a row
// is read from HBM exactly once and each output is written once. Row data and
// outputs move with non-temporal loads/stores (single use; dirty lines would
// otherwise be flushed from L2 at the end of the kernel); the weight vector,
// shared by every row, keeps the default cache policy. Rows up to
// 8 vectors per lane and 16 waves fit; wider rows or rows that are not a
// multiple of 8 elements, or unaligned buffers, use the element-wise kernel.
#include "ng_common.hpp"
#include "ng_exact.hpp"

namespace ng {

struct RowArgs {
    void* y;             // normed output [rows, H]            (NORM and !QUANT)
    void* res_out;       // residual output [rows, H]          (ADD)
    int8_t* q;           // int8 codes [rows, H]               (QUANT)
    float* scales;       // fp32 scale per row [rows]          (QUANT)
    const void* x;       // input [rows, H]
    const void* res;     // residual input [rows, H]           (ADD)
    const void* w;       // weight [H]                         (NORM)
    int H;
    int nvec;            // H / 8
    float eps;
};

template <int V>
struct MaxThreads {
    static constexpr int value = V <= 4 ? 1024 : 256;
};

template <typename T, int V, bool NORM, bool ADD, bool QUANT, bool WLATE>
__global__ __launch_bounds__(MaxThreads<V>::value) void row_kernel(RowArgs a) {
    static_assert(!WLATE || (NORM && !ADD && !QUANT), "late weights are for plain RMSNorm");
    __shared__ double s_part[16][3];
    __shared__ int s_flag[16];
    __shared__ uint32_t s_max[16];

    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int wid = tid >> 6;
    const int nw = nthr >> 6;
    const int lane = tid & 63;
    const size_t rowoff = static_cast<size_t>(blockIdx.x) * static_cast<size_t>(a.H);

    const uint16_t* xr = static_cast<const uint16_t*>(a.x) + rowoff;
    const uint16_t* rr = ADD ? static_cast<const uint16_t*>(a.res) + rowoff : nullptr;
    const uint16_t* wr = static_cast<const uint16_t*>(a.w);

    // All of the row's loads are issued before any arithmetic, unconditionally,
    // so that the reduction consumes each vector as it arrives. With
    // V = ceil(nvec / nthr) only the last vector of a lane can lie past the
    // row end: it is loaded from a clamped (valid) index, zeroed, and never
    // stored. A clamped load may read a vector another wave of the workgroup
    // later overwrites in place; that wave stores only after the workgroup
    // barrier of the reduction, by which point every load has been consumed.
    u32x4 xv[V], rv[V], wv[V];
    bool act[V];
#pragma unroll
    for (int k = 0; k < V; ++k) {
        const int vi = tid + k * nthr;
        act[k] = k < V - 1 || vi < a.nvec;
        const int vc = act[k] ? vi : a.nvec - 1;
        xv[k] = ld16_stream(xr + vc * 8);
        if (ADD) rv[k] = ld16_stream(rr + vc * 8);
    }
    // The weight row is the same for every row of the grid. Plain RMSNorm
    // over 2048 rows or more (WLATE) loads it only after the reduction:
    // issued at kernel start by every wave at once, these loads all land on
    // the same few L2 lines and slow the row loads behind them (measured on
    // MI355X: 13.3 vs 10.9 us for T = H = 4096). With fewer rows the second
    // memory round trip costs more than it saves (T = 64: 2.7 vs 2.4 us;
    // T = 1024: 4.8 vs 4.3 us), and the residual and quantising variants,
    // which have more work after the reduction, are faster with the weights
    // loaded early at every size.
    constexpr bool kWeightsLate = WLATE;
    if (NORM && !kWeightsLate) {
#pragma unroll
        for (int k = 0; k < V; ++k) {
            const int vi = tid + k * nthr;
            wv[k] = ld16(wr + (act[k] ? vi : a.nvec - 1) * 8);
        }
    }
    // Keep the scheduler from sinking any of these loads below the arithmetic.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < V; ++k) {
        if (!act[k]) {
            xv[k] = u32x4{0, 0, 0, 0};
            if (ADD) rv[k] = u32x4{0, 0, 0, 0};
        }
    }

    // o = the values the second pass scales: x, or the rounded residual sum.
    u32x4 ov[V];
    float r = 1.0f;
    if (NORM) {
        double acc[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int k = 0; k < V; ++k) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float s0, s1;
                if (ADD) {
                    s0 = el_add<T, 0>(xv[k][i], rv[k][i]);
                    s1 = el_add<T, 1>(xv[k][i], rv[k][i]);
                    ov[k][i] = pack2<T>(s0, s1);
                } else {
                    s0 = el_get<T, 0>(xv[k][i]);
                    s1 = el_get<T, 1>(xv[k][i]);
                    ov[k][i] = xv[k][i];
                }
                const double d0 = static_cast<double>(s0), d1 = static_cast<double>(s1);
                acc[(2 * i) & 3] = __builtin_fma(d0, d0, acc[(2 * i) & 3]);
                acc[(2 * i + 1) & 3] = __builtin_fma(d1, d1, acc[(2 * i + 1) & 3]);
            }
        }
        // Keep only the packed row live across the reduction: the second pass
        // converts again instead of holding 8 V unpacked floats.
#pragma unroll
        for (int k = 0; k < V; ++k) __asm__("" : "+v"(ov[k]));
        // S sums the squares in fp64. Plain RMSNorm with late weights combines
        // the lanes' and waves' partial sums with error-free transformations:
        // the extra arithmetic before its first store makes it faster
        // (measured on MI355X at T = H = 4096: 11.0 vs 11.45 us); the other
        // variants are faster without it.
        double S;
        if constexpr (kWeightsLate) {
            DD D2 = wave_sum_dd(dd_add(two_sum(acc[0], acc[1]), two_sum(acc[2], acc[3])));
            if (nw > 1) {
                if (lane == 0) {
                    s_part[wid][0] = D2.hi;
                    s_part[wid][1] = D2.lo;
                }
                __syncthreads();
                D2 = {s_part[0][0], s_part[0][1]};
                for (int j = 1; j < nw; ++j) D2 = dd_add(D2, DD{s_part[j][0], s_part[j][1]});
            }
            S = D2.hi;
        } else {
            S = wave_sum_f64_dpp((acc[0] + acc[1]) + (acc[2] + acc[3]));
            if (nw > 1) {
                if (lane == 0) s_part[wid][0] = S;
                __syncthreads();
                S = s_part[0][0];
                for (int j = 1; j < nw; ++j) S += s_part[j][0];
            }
        }
        // Error bound: with the error-free combination, that of one lane
        // accumulator (2 V terms); otherwise the height of the summation tree
        // (2 V terms per accumulator, 2 to join the four, 6 across the wave,
        // nw - 1 across waves).
        float ss;
        if (!ss_fast_resolve(S, kWeightsLate ? 2 * V : 2 * V + 8 + nw, ss)) {
            // Exact path (identical decision in every thread of the row). It
            // re-reads the row: nothing has been stored yet, so in-place
            // calls still see their inputs, and the registers above stay free.
            Limbs Lm{0.0, 0.0, 0.0, 0};
#pragma unroll 1
            for (int vi = tid; vi < a.nvec; vi += nthr) {
                float fx[8];
                unpack8<T>(ld16(xr + vi * 8), fx);
                if (ADD) {
                    float fr[8];
                    unpack8<T>(ld16(rr + vi * 8), fr);
#pragma unroll
                    for (int i = 0; i < 8; ++i) fx[i] = fx[i] + fr[i];
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) limbs_add(Lm, fx[i]);
            }
            // Limb sums are exact integers: any summation order gives the same bits.
            double t = wave_sum_f64_dpp(Lm.t), u = wave_sum_f64_dpp(Lm.u), w = wave_sum_f64_dpp(Lm.w);
            int bad = static_cast<int>(wave_max_u32_dpp(static_cast<uint32_t>(Lm.bad)));
            if (nw > 1) {
                __syncthreads();
                if (lane == 0) {
                    s_part[wid][0] = t;
                    s_part[wid][1] = u;
                    s_part[wid][2] = w;
                    s_flag[wid] = bad;
                }
                __syncthreads();
                t = u = w = 0.0;
                bad = 0;
                for (int j = 0; j < nw; ++j) {
                    t += s_part[j][0];
                    u += s_part[j][1];
                    w += s_part[j][2];
                    bad |= s_flag[j];
                }
            }
            if (!bad) ss = limbs_to_f32(t, u, w);
        }
        r = 1.0f / __builtin_sqrtf(ss / static_cast<float>(a.H) + a.eps);
        if (ADD) {
#pragma unroll
            for (int k = 0; k < V; ++k)
                if (act[k]) st16_stream(static_cast<uint16_t*>(a.res_out) + rowoff + (tid + k * nthr) * 8, ov[k]);
        }
    } else {
#pragma unroll
        for (int k = 0; k < V; ++k) ov[k] = xv[k];
    }

    // Second pass: y = RN_T(RN(o * r) * w), or v = x when only quantising.
    if (kWeightsLate) {
#pragma unroll
        for (int k = 0; k < V; ++k) {
            const int vi = tid + k * nthr;
            wv[k] = ld16(wr + (act[k] ? vi : a.nvec - 1) * 8);
        }
    }
    u32x4 yv[V];
    if (NORM) {
#pragma unroll
        for (int k = 0; k < V; ++k) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float y0 = el_mul<T, 0>(wv[k][i], el_mul<T, 0>(ov[k][i], r));
                const float y1 = el_mul<T, 1>(wv[k][i], el_mul<T, 1>(ov[k][i], r));
                yv[k][i] = pack2<T>(y0, y1);
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < V; ++k) yv[k] = xv[k];
    }

    if (!QUANT) {
        uint16_t* yr = static_cast<uint16_t*>(a.y) + rowoff;
#pragma unroll
        for (int k = 0; k < V; ++k)
            if (act[k]) st16_stream(yr + (tid + k * nthr) * 8, yv[k]);
        return;
    }

    // Row absmax on the 16-bit patterns (inactive vectors hold zeros).
    uint32_t mx = 0;
#pragma unroll
    for (int k = 0; k < V; ++k) mx = absmax_bits8(act[k] ? yv[k] : u32x4{0, 0, 0, 0}, mx);
    mx = wave_max_u32_dpp(mx);
    if (nw > 1) {
        if (lane == 0) s_max[wid] = mx;
        __syncthreads();
        mx = 0;
        for (int j = 0; j < nw; ++j) mx = umax32(mx, s_max[j]);
    }
    // A row holding a NaN (uniform over the workgroup): the maximum again,
    // without the NaNs, as the reference's fmaxf reduction takes it.
    const bool has_nan = mx > kInfBits<T>;
    if (has_nan) {
        __shared__ uint32_t s_max2[16];
        mx = 0;
#pragma unroll
        for (int k = 0; k < V; ++k) mx = absmax_bits8_nonan<T>(act[k] ? yv[k] : u32x4{0, 0, 0, 0}, mx);
        mx = wave_max_u32_dpp(mx);
        if (nw > 1) {
            if (lane == 0) s_max2[wid] = mx;
            __syncthreads();
            mx = 0;
            for (int j = 0; j < nw; ++j) mx = umax32(mx, s_max2[j]);
        }
    }
    const float m = to_f32<T>(static_cast<uint16_t>(mx));
    float scale = m / 127.0f;
    if (scale == 0.0f) scale = 1.0f;
    const float inv = 1.0f / scale;
    if (tid == 0) a.scales[blockIdx.x] = scale;

    int8_t* qr = a.q + rowoff;
    const bool fast = !has_nan && __builtin_isfinite(scale);  // uniform over the row
#pragma unroll
    for (int k = 0; k < V; ++k) {
        const u32x2 c = fast ? qcode8<T>(yv[k], inv, -scale) : qcode8_div<T>(yv[k], scale);
        if (act[k]) __builtin_nontemporal_store(c, reinterpret_cast<u32x2*>(qr + (tid + k * nthr) * 8));
    }
}

// RN_f32 of the exact sum of squares of one row held by a single wave,
// recomputed from memory with the 3-limb integer method (ng_exact.hpp): the
// fallback of the fp64 fast path. Returns false (ss untouched) for rows with
// a value off the 2^-24 grid.
template <typename T, bool ADD>
__device__ __forceinline__ bool exact_row_ss_wave(const uint16_t* xr, const uint16_t* rr, int nvec, int lane, float& ss) {
    Limbs Lm{0.0, 0.0, 0.0, 0};
    for (int vi = lane; vi < nvec; vi += kWave) {
        float fx[8];
        unpack8<T>(ld16(xr + vi * 8), fx);
        if (ADD) {
            float fr[8];
            unpack8<T>(ld16(rr + vi * 8), fr);
#pragma unroll
            for (int i = 0; i < 8; ++i) fx[i] = fx[i] + fr[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) limbs_add(Lm, fx[i]);
    }
    const double t = wave_sum_f64_dpp(Lm.t), u = wave_sum_f64_dpp(Lm.u), w = wave_sum_f64_dpp(Lm.w);
    if (wave_max_u32_dpp(static_cast<uint32_t>(Lm.bad))) return false;
    ss = limbs_to_f32(t, u, w);
    return true;
}

// Residual add + RMSNorm for rows that fit one wave (nvec <= 64 V), R rows
// per wave: the loads of all R rows are issued first, then each row is
// reduced, normalised and stored in turn, so the stores of the first rows
// overlap the arrival of the later ones. Same arithmetic as row_kernel.
// Rows past the last one are loaded from the last row and never stored.
template <typename T, int V, int R>
__global__ __launch_bounds__(64) void add_rms_rows_kernel(RowArgs a, int rows) {
    const int lane = threadIdx.x;
    const int row0 = blockIdx.x * R;
    const uint16_t* X = static_cast<const uint16_t*>(a.x);
    const uint16_t* RS = static_cast<const uint16_t*>(a.res);
    const uint16_t* wr = static_cast<const uint16_t*>(a.w);
    bool act[V];
    int vc[V];
#pragma unroll
    for (int k = 0; k < V; ++k) {
        const int vi = lane + k * kWave;
        act[k] = k < V - 1 || vi < a.nvec;
        vc[k] = act[k] ? vi : a.nvec - 1;
    }
    u32x4 xv[R][V], rv[R][V], wv[V];
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const size_t off = static_cast<size_t>(min(row0 + j, rows - 1)) * a.H;
#pragma unroll
        for (int k = 0; k < V; ++k) {
            xv[j][k] = ld16_stream(X + off + vc[k] * 8);
            rv[j][k] = ld16_stream(RS + off + vc[k] * 8);
        }
    }
    // The weight row is read by every wave. With four rows per wave it is
    // loaded once the first row's statistic is known: issued with the row
    // loads, these loads of the same few lines slowed them (measured on
    // MI355X at T = H = 4096, in place: 22.0 us against 22.75 us), as in plain
    // RMSNorm. With two rows per wave (H = 5120) loading it up front is faster
    // (T = 2048, bf16: 14.55 us against 15.05 us).
    constexpr bool kWeightsLate = R >= 4;
    if (!kWeightsLate) {
#pragma unroll
        for (int k = 0; k < V; ++k) wv[k] = ld16(wr + vc[k] * 8);
    }
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int j = 0; j < R; ++j) {
        if (row0 + j >= rows) break;
        const size_t off = static_cast<size_t>(row0 + j) * a.H;
        u32x4 ov[V];
        double acc[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int k = 0; k < V; ++k) {
            if (!act[k]) {
                xv[j][k] = u32x4{0, 0, 0, 0};
                rv[j][k] = u32x4{0, 0, 0, 0};
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float s0 = el_add<T, 0>(xv[j][k][i], rv[j][k][i]);
                const float s1 = el_add<T, 1>(xv[j][k][i], rv[j][k][i]);
                ov[k][i] = pack2<T>(s0, s1);
                const double d0 = static_cast<double>(s0), d1 = static_cast<double>(s1);
                acc[(2 * i) & 3] = __builtin_fma(d0, d0, acc[(2 * i) & 3]);
                acc[(2 * i + 1) & 3] = __builtin_fma(d1, d1, acc[(2 * i + 1) & 3]);
            }
        }
        const double S = wave_sum_f64_dpp((acc[0] + acc[1]) + (acc[2] + acc[3]));
        float ss;
        // Summation tree height: 2 V per accumulator, 2 to join them, 6 across the wave.
        if (!ss_fast_resolve(S, 2 * V + 8, ss)) exact_row_ss_wave<T, true>(X + off, RS + off, a.nvec, lane, ss);
        const float r = 1.0f / __builtin_sqrtf(ss / static_cast<float>(a.H) + a.eps);
        if (kWeightsLate && j == 0) {
#pragma unroll
            for (int k = 0; k < V; ++k) wv[k] = ld16(wr + vc[k] * 8);
        }
        uint16_t* ro = static_cast<uint16_t*>(a.res_out) + off;
        uint16_t* yr = static_cast<uint16_t*>(a.y) + off;
#pragma unroll
        for (int k = 0; k < V; ++k)
            if (act[k]) st16_stream(ro + (lane + k * kWave) * 8, ov[k]);
#pragma unroll
        for (int k = 0; k < V; ++k) {
            u32x4 y;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                y[i] = pack2<T>(el_mul<T, 0>(wv[k][i], el_mul<T, 0>(ov[k][i], r)),
                                el_mul<T, 1>(wv[k][i], el_mul<T, 1>(ov[k][i], r)));
            if (act[k]) st16_stream(yr + (lane + k * kWave) * 8, y);
        }
    }
}

// Element-wise fallback for any H and any alignment: one workgroup per row,
// the row re-read from memory for each pass. Same arithmetic as row_kernel.
template <typename T, bool NORM, bool ADD, bool QUANT>
__global__ __launch_bounds__(256) void row_kernel_scalar(RowArgs a) {
    __shared__ double s_part[4][3];
    __shared__ int s_flag[4];
    __shared__ uint32_t s_max[4];
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int wid = tid >> 6, nw = nthr >> 6, lane = tid & 63;
    const size_t rowoff = static_cast<size_t>(blockIdx.x) * static_cast<size_t>(a.H);
    const uint16_t* xr = static_cast<const uint16_t*>(a.x) + rowoff;
    const uint16_t* rr = ADD ? static_cast<const uint16_t*>(a.res) + rowoff : nullptr;
    const uint16_t* wr = static_cast<const uint16_t*>(a.w);

    auto sval = [&](int i) -> float {
        float v = to_f32<T>(xr[i]);
        if (ADD) v = v + to_f32<T>(rr[i]);
        return v;
    };

    float r = 1.0f;
    if (NORM) {
        double acc = 0.0;
        for (int i = tid; i < a.H; i += nthr) {
            const double d = static_cast<double>(sval(i));
            acc = __builtin_fma(d, d, acc);
        }
        DD S = wave_sum_dd(DD{acc, 0.0});
        if (lane == 0) {
            s_part[wid][0] = S.hi;
            s_part[wid][1] = S.lo;
        }
        __syncthreads();
        S = {s_part[0][0], s_part[0][1]};
        for (int j = 1; j < nw; ++j) S = dd_add(S, DD{s_part[j][0], s_part[j][1]});
        float ss;
        if (!ss_fast_resolve(S.hi, (a.H + nthr - 1) / nthr, ss)) {
            Limbs Lm{0.0, 0.0, 0.0, 0};
            for (int i = tid; i < a.H; i += nthr) limbs_add(Lm, sval(i));
            double t = wave_sum_f64_dpp(Lm.t), u = wave_sum_f64_dpp(Lm.u), w = wave_sum_f64_dpp(Lm.w);
            int bad = static_cast<int>(wave_max_u32_dpp(static_cast<uint32_t>(Lm.bad)));
            __syncthreads();
            if (lane == 0) {
                s_part[wid][0] = t;
                s_part[wid][1] = u;
                s_part[wid][2] = w;
                s_flag[wid] = bad;
            }
            __syncthreads();
            t = u = w = 0.0;
            bad = 0;
            for (int j = 0; j < nw; ++j) {
                t += s_part[j][0];
                u += s_part[j][1];
                w += s_part[j][2];
                bad |= s_flag[j];
            }
            if (!bad) ss = limbs_to_f32(t, u, w);
        }
        r = 1.0f / __builtin_sqrtf(ss / static_cast<float>(a.H) + a.eps);
    }

    // v_i as the 16-bit pattern that is stored or quantised.
    auto vbits = [&](int i) -> uint16_t {
        if (!NORM) return xr[i];
        float o = ADD ? to_f32<T>(from_f32<T>(sval(i))) : to_f32<T>(xr[i]);
        return from_f32<T>((o * r) * to_f32<T>(wr[i]));
    };

    if (!QUANT) {
        uint16_t* yr = static_cast<uint16_t*>(a.y) + rowoff;
        uint16_t* ror = ADD ? static_cast<uint16_t*>(a.res_out) + rowoff : nullptr;
        for (int i = tid; i < a.H; i += nthr) {
            // Both values are computed before either store: the outputs may
            // alias the inputs element for element.
            const uint16_t yb = vbits(i);
            const uint16_t rb = ADD ? from_f32<T>(sval(i)) : 0;
            if (ADD) ror[i] = rb;
            yr[i] = yb;
        }
        return;
    }

    uint32_t mx = 0;
    for (int i = tid; i < a.H; i += nthr) {
        const uint32_t b = absbits_nonan<T>(vbits(i));  // NaNs skipped, as fmaxf does
        mx = mx > b ? mx : b;
    }
    mx = wave_max_u32_dpp(mx);
    if (lane == 0) s_max[wid] = mx;
    __syncthreads();
    mx = 0;
    for (int j = 0; j < nw; ++j) mx = mx > s_max[j] ? mx : s_max[j];
    const float m = to_f32<T>(static_cast<uint16_t>(mx));
    float scale = m / 127.0f;
    if (scale == 0.0f) scale = 1.0f;
    const float inv = 1.0f / scale;
    if (tid == 0) a.scales[blockIdx.x] = scale;
    int8_t* qr = a.q + rowoff;
    uint16_t* ror = ADD ? static_cast<uint16_t*>(a.res_out) + rowoff : nullptr;
    for (int i = tid; i < a.H; i += nthr) {
        const uint16_t vb = vbits(i);
        const uint16_t rb = ADD ? from_f32<T>(sval(i)) : 0;
        if (ADD) ror[i] = rb;
        qr[i] = static_cast<int8_t>(qcode_int(to_f32<T>(vb), scale, inv));
    }
}

// ---------------------------------------------------------------------------
// Host dispatch.
// ---------------------------------------------------------------------------
template <typename T, bool NORM, bool ADD, bool QUANT>
struct RowDispatch {
    template <int V>
    static void go(dim3 g, dim3 b, const RowArgs& a, bool late) {
        if constexpr (NORM && !ADD && !QUANT) {
            if (late) {
                row_kernel<T, V, NORM, ADD, QUANT, true><<<g, b, 0, stream()>>>(a);
                return;
            }
        }
        row_kernel<T, V, NORM, ADD, QUANT, false><<<g, b, 0, stream()>>>(a);
    }
    static bool launch(int V, dim3 g, dim3 b, const RowArgs& a, bool late) {
        switch (V) {
            case 1: go<1>(g, b, a, late); return true;
            case 2: go<2>(g, b, a, late); return true;
            case 3: go<3>(g, b, a, late); return true;
            case 4: go<4>(g, b, a, late); return true;
            case 5: go<5>(g, b, a, late); return true;
            case 6: go<6>(g, b, a, late); return true;
            case 7: go<7>(g, b, a, late); return true;
            case 8: go<8>(g, b, a, late); return true;
            default: return false;
        }
    }
};

// Workgroup shape for a row of nvec 16-byte vectors: returns false when the
// row does not fit in registers.
static bool pick_row_shape(int nvec, int rows, int& nw, int& V) {
    // Many rows: few waves per row, more vectors in flight per lane. Few
    // rows (decode): spread each row over more waves.
    int target_v = rows >= 2048 ? 8 : (rows >= 512 ? 4 : 2);
    nw = (nvec + 64 * target_v - 1) / (64 * target_v);
    if (nw < 1) nw = 1;
    if (nw > 16) nw = 16;
    V = (nvec + 64 * nw - 1) / (64 * nw);
    if (V > 4 && nw > 4) {
        nw = 16;
        V = (nvec + 64 * nw - 1) / (64 * nw);
    }
    return V >= 1 && V <= 8 && !(V > 4 && nw > 4);
}

template <typename T, bool NORM, bool ADD, bool QUANT>
static int launch_rows(const char* name, int rows, const RowArgs& a0) {
    RowArgs a = a0;
    a.nvec = a.H / 8;
    bool vec_ok = (a.H % 8 == 0) && aligned16(a.x) && (!ADD || aligned16(a.res)) &&
                  (!ADD || aligned16(a.res_out)) && (!NORM || aligned16(a.w)) &&
                  (QUANT || !NORM || aligned16(a.y)) && (!QUANT || aligned8(a.q));
    int nw = 0, V = 0;
    if (vec_ok && pick_row_shape(a.nvec, rows, nw, V)) {
        if constexpr (NORM && ADD && !QUANT) {
            // Residual add + RMSNorm at prefill sizes, shapes measured on MI355X.
            // Several rows per wave pays when it leaves about 1024 waves (one per
            // SIMD), each with many bytes in flight:
            //   H = 4096, T >= 4096: 4 rows per wave      (T = 4096: 22.8 vs 24.0 us)
            //   H = 5120, T in [1536, 4096): 2 rows/wave  (T = 2048: 14.5 vs 15.9 us)
            // The engine's in-place aliasing (layer.cu:1038) is safe: a row's
            // stores come after that row's loads, and no two waves share a row.
            if (a.nvec == 512 && rows >= 4096) {
                add_rms_rows_kernel<T, 8, 4><<<dim3((rows + 3) / 4), dim3(64), 0, stream()>>>(a, rows);
                NG_CHECK_LAUNCH(name);
                return 0;
            }
            if (a.nvec == 640 && rows >= 1536 && rows < 4096) {
                add_rms_rows_kernel<T, 10, 2><<<dim3((rows + 1) / 2), dim3(64), 0, stream()>>>(a, rows);
                NG_CHECK_LAUNCH(name);
                return 0;
            }
            //   H = 5120, T >= 4096: 5 waves of 2 vectors per lane (T = 8192, in
            //   place: 54.96 vs 56.02 us with 2 waves of 5, 55.77 with 4 of 3)
            if (a.nvec == 640 && rows >= 4096) {
                nw = 5;
                V = 2;
            }
        }
        // Per-row int8 quantisation alone (no statistic to compute) over
        // rows of 4096: two waves of 4 vectors per row (measured on MI355X at
        // T = 4096: 10.08 vs 10.33 us with one wave of 8; the fused norm + int8
        // kernels are slower with two).
        if (QUANT && !NORM && rows >= 2048 && a.nvec == 512) {
            nw = 2;
            V = 4;
        }
        RowDispatch<T, NORM, ADD, QUANT>::launch(V, dim3(rows), dim3(nw * 64), a, rows >= 2048);
    } else {
        row_kernel_scalar<T, NORM, ADD, QUANT><<<dim3(rows), dim3(256), 0, stream()>>>(a);
    }
    NG_CHECK_LAUNCH(name);
    return 0;
}

}  // namespace ng

using namespace ng;

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" int cuda_rmsnorm(void* output, const void* input, const void* weight,
                            int num_tokens, int hidden_dim, float eps) {
    NG_REQUIRE(output && input && weight, "cuda_rmsnorm: null pointer");
    NG_REQUIRE(num_tokens > 0 && hidden_dim > 0, "cuda_rmsnorm: num_tokens=%d hidden_dim=%d must be > 0",
               num_tokens, hidden_dim);
    RowArgs a{};
    a.y = output; a.x = input; a.w = weight; a.H = hidden_dim; a.eps = eps;
    return launch_rows<f16, true, false, false>("cuda_rmsnorm", num_tokens, a);
}

extern "C" int cuda_bf16_rmsnorm(void* output, const void* input, const void* weight,
                                 int num_tokens, int hidden_dim, float eps) {
    NG_REQUIRE(output && input && weight, "cuda_bf16_rmsnorm: null pointer");
    NG_REQUIRE(num_tokens > 0 && hidden_dim > 0, "cuda_bf16_rmsnorm: num_tokens=%d hidden_dim=%d must be > 0",
               num_tokens, hidden_dim);
    RowArgs a{};
    a.y = output; a.x = input; a.w = weight; a.H = hidden_dim; a.eps = eps;
    return launch_rows<bf16, true, false, false>("cuda_bf16_rmsnorm", num_tokens, a);
}

extern "C" int cuda_add_rmsnorm(void* normed_output, void* residual_output, const void* input,
                                const void* residual_input, const void* weight, int num_tokens,
                                int hidden_dim, float eps) {
    NG_REQUIRE(normed_output && residual_output && input && residual_input && weight,
               "cuda_add_rmsnorm: null pointer");
    NG_REQUIRE(num_tokens > 0 && hidden_dim > 0, "cuda_add_rmsnorm: num_tokens=%d hidden_dim=%d must be > 0",
               num_tokens, hidden_dim);
    RowArgs a{};
    a.y = normed_output; a.res_out = residual_output; a.x = input; a.res = residual_input;
    a.w = weight; a.H = hidden_dim; a.eps = eps;
    return launch_rows<f16, true, true, false>("cuda_add_rmsnorm", num_tokens, a);
}

extern "C" int ng_bf16_add_rmsnorm(void* normed_output, void* residual_output, const void* input,
                                   const void* residual_input, const void* weight, int num_tokens,
                                   int hidden_dim, float eps) {
    NG_REQUIRE(normed_output && residual_output && input && residual_input && weight,
               "ng_bf16_add_rmsnorm: null pointer");
    NG_REQUIRE(num_tokens > 0 && hidden_dim > 0, "ng_bf16_add_rmsnorm: num_tokens=%d hidden_dim=%d must be > 0",
               num_tokens, hidden_dim);
    RowArgs a{};
    a.y = normed_output; a.res_out = residual_output; a.x = input; a.res = residual_input;
    a.w = weight; a.H = hidden_dim; a.eps = eps;
    return launch_rows<bf16, true, true, false>("ng_bf16_add_rmsnorm", num_tokens, a);
}

extern "C" int ng_rmsnorm_quant_int8(void* q_out, void* scales_out, const void* input,
                                     const void* weight, int num_tokens, int hidden_dim, float eps) {
    NG_REQUIRE(q_out && scales_out && input && weight, "ng_rmsnorm_quant_int8: null pointer");
    NG_REQUIRE(num_tokens > 0 && hidden_dim > 0, "ng_rmsnorm_quant_int8: num_tokens=%d hidden_dim=%d must be > 0",
               num_tokens, hidden_dim);
    RowArgs a{};
    a.q = static_cast<int8_t*>(q_out); a.scales = static_cast<float*>(scales_out);
    a.x = input; a.w = weight; a.H = hidden_dim; a.eps = eps;
    return launch_rows<f16, true, false, true>("ng_rmsnorm_quant_int8", num_tokens, a);
}

extern "C" int ng_add_rmsnorm_quant_int8(void* q_out, void* scales_out, void* residual_output,
                                         const void* input, const void* residual_input,
                                         const void* weight, int num_tokens, int hidden_dim,
                                         float eps) {
    NG_REQUIRE(q_out && scales_out && residual_output && input && residual_input && weight,
               "ng_add_rmsnorm_quant_int8: null pointer");
    NG_REQUIRE(num_tokens > 0 && hidden_dim > 0,
               "ng_add_rmsnorm_quant_int8: num_tokens=%d hidden_dim=%d must be > 0", num_tokens, hidden_dim);
    RowArgs a{};
    a.q = static_cast<int8_t*>(q_out); a.scales = static_cast<float*>(scales_out);
    a.res_out = residual_output; a.x = input; a.res = residual_input;
    a.w = weight; a.H = hidden_dim; a.eps = eps;
    return launch_rows<f16, true, true, true>("ng_add_rmsnorm_quant_int8", num_tokens, a);
}

extern "C" int cuda_quantize_weights_per_row(void* output, void* scales, const void* input,
                                             int rows, int cols) {
    NG_REQUIRE(output && scales && input, "cuda_quantize_weights_per_row: null pointer");
    NG_REQUIRE(rows > 0 && cols > 0, "cuda_quantize_weights_per_row: rows=%d cols=%d must be > 0", rows, cols);
    RowArgs a{};
    a.q = static_cast<int8_t*>(output); a.scales = static_cast<float*>(scales);
    a.x = input; a.H = cols;
    return launch_rows<f16, false, false, true>("cuda_quantize_weights_per_row", rows, a);
}

namespace ng {

// RMSNorm of `rows` rows of H elements through the row kernels, for the
// per-head RMSNorm's fallback (rope.hip).
template <typename T>
int rows_rmsnorm(const char* name, void* output, const void* input, const void* weight, int rows, int H,
                 float eps) {
    RowArgs a{};
    a.y = output; a.x = input; a.w = weight; a.H = H; a.eps = eps;
    return launch_rows<T, true, false, false>(name, rows, a);
}

template int rows_rmsnorm<f16>(const char*, void*, const void*, const void*, int, int, float);
template int rows_rmsnorm<bf16>(const char*, void*, const void*, const void*, int, int, float);

}  // namespace ng
