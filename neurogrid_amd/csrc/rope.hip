// rope.hip - rotary position embedding on [batch, seq, heads, head_dim].
//
// Semantics (reference: gpu/cuda/kernels.cu:431-489, bf16_utils.cu:330-378):
//   inv_i = 1 / powf(theta, (2 i) / D)         i < D/2, computed on the host
//   a     = float(pos[t]) * inv_i               one fp32 rounding
//   (c, s)= (cos a, sin a)                      accurate sincosf
//   x1' = x1 c - x2 s,  x2' = x1 s + x2 c       rounded once to the element type
//   split-half pairs (i, i + D/2); interleaved pairs (2i, 2i + 1)
//
// The angle depends on (token, pair) only. A workgroup takes a tile of tokens,
// evaluates each of its tile * D/2 (cos, sin) pairs once into LDS, then
// rotates every head of those tokens with 16-byte vector accesses; the
// reference evaluates powf/sincos again for every head.
#include "ng_common.hpp"
#include "ng_exact.hpp"
#include "../../include/neurogrid_ext.h"

#include <math.h>

#include <mutex>
#include <unordered_map>
#include <vector>

namespace ng {

constexpr int kRopeThreads = 256;
constexpr int kRopeMaxHalf = 128;  // D <= 256

struct RopeArgs {
    void* out;
    const void* in;
    const int* pos;
    int T;             // tokens
    int nh;            // heads
    int D;             // head_dim
    int half;          // D / 2
    int upt;           // work units per token
    int units;         // T * upt
    FastDiv div_upt;   // divide by units per token
    FastDiv div_uph;   // divide by units per head
    FastDiv div_half;  // divide by D / 2
    float inv_freq[kRopeMaxHalf];
};

// A work unit is one 16-byte vector of a head (interleaved style: pairs
// [4j, 4j+4) at offset 8j) or a matching pair of vectors (split-half style:
// pairs [8j, 8j+8) at offsets 8j and D/2 + 8j). A workgroup takes U * 256
// consecutive units, i.e. a run of consecutive tokens:
//   1. issue every global load of its units;
//   2. while they are in flight, evaluate (cos, sin) once per (token, pair)
//      of its tokens into LDS;
//   3. rotate and store.
template <typename T, int STYLE, int U>
__global__ __launch_bounds__(kRopeThreads) void rope_vec_kernel(RopeArgs a) {
    extern __shared__ float2 cs[];  // [tokens of this workgroup][half]
    const int u0 = blockIdx.x * (kRopeThreads * U);
    const int ulast = min(u0 + kRopeThreads * U, a.units) - 1;
    const int tfirst = static_cast<int>(fdiv(static_cast<uint32_t>(u0), a.div_upt));
    const int ntok = static_cast<int>(fdiv(static_cast<uint32_t>(ulast), a.div_upt)) - tfirst + 1;
    const uint16_t* in = static_cast<const uint16_t*>(a.in);
    uint16_t* out = static_cast<uint16_t*>(a.out);

    u32x4 v1[U], v2[U];
    size_t base[U];
    int tl[U], jj[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const int u = u0 + k * kRopeThreads + static_cast<int>(threadIdx.x);
        const int uc = u < a.units ? u : ulast;
        const int t = static_cast<int>(fdiv(static_cast<uint32_t>(uc), a.div_upt));
        const int rem = uc - t * a.upt;
        const int h = static_cast<int>(fdiv(static_cast<uint32_t>(rem), a.div_uph));
        jj[k] = rem - h * static_cast<int>(a.div_uph.d);
        tl[k] = t - tfirst;
        base[k] = (static_cast<size_t>(t) * a.nh + h) * a.D + 8 * jj[k];
        v1[k] = ld16_stream(in + base[k]);
        if (STYLE == 0) v2[k] = ld16_stream(in + base[k] + a.half);
    }

    const int ncs = ntok * a.half;
    for (int idx = threadIdx.x; idx < ncs; idx += kRopeThreads) {
        const int t = static_cast<int>(fdiv(static_cast<uint32_t>(idx), a.div_half));
        const int i = idx - t * a.half;
        const float ang = static_cast<float>(a.pos[tfirst + t]) * a.inv_freq[i];
        float sn, c;
        sincosf(ang, &sn, &c);
        cs[idx] = make_float2(c, sn);
    }
    __syncthreads();

#pragma unroll
    for (int k = 0; k < U; ++k) {
        const int u = u0 + k * kRopeThreads + static_cast<int>(threadIdx.x);
        if (u >= a.units) break;
        const float2* c = cs + tl[k] * a.half;
        if (STYLE == 0) {
            float x1[8], x2[8], y1[8], y2[8];
            unpack8<T>(v1[k], x1);
            unpack8<T>(v2[k], x2);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float2 q = c[8 * jj[k] + e];
                y1[e] = x1[e] * q.x - x2[e] * q.y;
                y2[e] = x1[e] * q.y + x2[e] * q.x;
            }
            st16_stream(out + base[k], pack8<T>(y1));
            st16_stream(out + base[k] + a.half, pack8<T>(y2));
        } else {
            float x[8], y[8];
            unpack8<T>(v1[k], x);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float2 q = c[4 * jj[k] + e];
                y[2 * e] = x[2 * e] * q.x - x[2 * e + 1] * q.y;
                y[2 * e + 1] = x[2 * e] * q.y + x[2 * e + 1] * q.x;
            }
            st16_stream(out + base[k], pack8<T>(y));
        }
    }
}

// Wave-per-token kernel, for head_dim 64, 128 or 256 (16-byte aligned).
// A wave rotates HPL passes of heads of one token; a pass covers 64 / lph
// heads, lph lanes per head (split-half: lane j of a head owns vector j of
// each half, pairs 8j..8j+7; interleaved: vector j, pairs 4j..4j+3). Lane l
// evaluates (cos, sin) of pairs l and l + 64 once; the lanes that need them
// fetch them with cross-lane shuffles, so each (token, pair) angle is
// evaluated once per wave, with no LDS table and no workgroup barrier. All
// loads are issued first, from clamped indices where a pass runs past the
// last head; those vectors are not stored. When T is small, a token's passes
// are split over G waves so that enough waves are in flight.
struct RopeWaveArgs {
    void* out;         // first tensor [T, nh, D]
    const void* in;
    void* out2;        // optional second tensor [T, nh2, D], same positions (nh2 = 0: none)
    const void* in2;
    const int* pos;
    int T;
    int nh;
    int nh2;
    int npass1;        // head passes of the first tensor; passes beyond it cover the second
    int D;
    int lph_log2;      // log2(lanes per head)
    int G;             // waves per token
    FastDiv div_G;
    const void* w1;    // per-head RMSNorm weights [D] of the first / second tensor (QKNORM)
    const void* w2;
    float eps;
    int dev_store;     // 1: device-scope stores (small in-place updates), 0: non-temporal
    float inv_freq[kRopeMaxHalf];
};

// Sums over the lph consecutive lanes that hold one head (lph a power of two
// up to 32). Each step adds the value of a partner lane in the complementary
// half of the current group, so every lane of the group ends with the same
// bits (fp64 addition is commutative bit for bit).
__device__ __forceinline__ double group_sum_f64(double v, int lph) {
    if (lph > 1) v += dpp_f64<kDppQuadSwap1>(v);
    if (lph > 2) v += dpp_f64<kDppQuadSwap2>(v);
    if (lph > 4) v += dpp_f64<kDppRowHalfMirror>(v);
    if (lph > 8) v += dpp_f64<kDppRowMirror>(v);
    if (lph > 16) v += __shfl_xor(v, 16, kWave);
    return v;
}

// Per-head RMSNorm of the NV 16-byte vectors a lane holds of one head (the
// head spread over lph lanes), in place: y = RN_T(RN(x * r) * w),
// r = 1 / sqrt(RN_f32(exact sum x^2) / D + eps), as the row kernels compute it.
template <typename T, int NV>
__device__ __forceinline__ void head_rmsnorm(u32x4 (&x)[NV], const u32x4 (&w)[NV], int lph, int D, float eps) {
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int n = 0; n < NV; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const double d0 = static_cast<double>(el_get<T, 0>(x[n][i]));
            const double d1 = static_cast<double>(el_get<T, 1>(x[n][i]));
            acc[(2 * i) & 3] = __builtin_fma(d0, d0, acc[(2 * i) & 3]);
            acc[(2 * i + 1) & 3] = __builtin_fma(d1, d1, acc[(2 * i + 1) & 3]);
        }
    const double S = group_sum_f64((acc[0] + acc[1]) + (acc[2] + acc[3]), lph);
    float ss;
    // Summation tree height: 2 NV per accumulator, 2 to join them, log2(lph) <= 5 across the head's lanes.
    if (!ss_fast_resolve(S, 2 * NV + 8, ss)) {
        // Exact path for this head (the whole lane group takes it together).
        Limbs Lm{0.0, 0.0, 0.0, 0};
#pragma unroll
        for (int n = 0; n < NV; ++n)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                limbs_add(Lm, el_get<T, 0>(x[n][i]));
                limbs_add(Lm, el_get<T, 1>(x[n][i]));
            }
        const double t = group_sum_f64(Lm.t, lph), u = group_sum_f64(Lm.u, lph), wl = group_sum_f64(Lm.w, lph);
        const double bad = group_sum_f64(static_cast<double>(Lm.bad), lph);
        if (bad == 0.0) ss = limbs_to_f32(t, u, wl);
    }
    const float r = 1.0f / __builtin_sqrtf(ss / static_cast<float>(D) + eps);
#pragma unroll
    for (int n = 0; n < NV; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            x[n][i] = pack2<T>(el_mul<T, 0>(w[n][i], el_mul<T, 0>(x[n][i], r)),
                               el_mul<T, 1>(w[n][i], el_mul<T, 1>(x[n][i], r)));
}

template <typename T, int STYLE, int HPL, bool QKNORM, bool ROT = true, bool EARLY = false>
__global__ __launch_bounds__(kRopeThreads) void rope_wave_kernel(RopeWaveArgs a) {
    static_assert(!EARLY || (ROT && !QKNORM), "early angles are for plain RoPE");
    const int lane = threadIdx.x & 63;
    // The wave index is uniform. With QK-norm, saying so makes the position
    // load a scalar load, which does not wait behind the head loads; plain
    // RoPE keeps the vector load, whose wait for every head it relies on
    // (below).
    const uint32_t wv = threadIdx.x >> 6;
    const uint32_t w = blockIdx.x * (blockDim.x >> 6) + (QKNORM ? __builtin_amdgcn_readfirstlane(wv) : wv);
    const int t = static_cast<int>(fdiv(w, a.div_G));
    if (t >= a.T) return;
    const int g = static_cast<int>(w) - t * a.G;
    const int lph = 1 << a.lph_log2;
    const int hpp = kWave >> a.lph_log2;
    const int j = lane & (lph - 1);
    const int hl = lane >> a.lph_log2;
    const int half = a.D >> 1;
    const uint16_t* in1 = static_cast<const uint16_t*>(a.in) + static_cast<size_t>(t) * a.nh * a.D;
    uint16_t* out1 = static_cast<uint16_t*>(a.out) + static_cast<size_t>(t) * a.nh * a.D;
    const uint16_t* in2 = static_cast<const uint16_t*>(a.in2) + static_cast<size_t>(t) * a.nh2 * a.D;
    uint16_t* out2 = static_cast<uint16_t*>(a.out2) + static_cast<size_t>(t) * a.nh2 * a.D;
    // Store of the vector at element offset `o` within this token's heads of
    // the first or second tensor. Device-scope stores (tensors of at most
    // 8 MiB) go through a buffer resource based at the tensor, with the
    // token's offset in the vector offset.
    // (`second` is the same for the whole wave; readfirstlane says so, which
    // keeps the resource in scalar registers.)
    auto store = [&](bool second_lane, uint32_t o, u32x4 v) {
        if (a.dev_store) {
            const bool second = __builtin_amdgcn_readfirstlane(static_cast<int>(second_lane)) != 0;
            const uint32_t nhs = static_cast<uint32_t>(second ? a.nh2 : a.nh);
            const uint32_t bytes = static_cast<uint32_t>(a.T) * nhs * static_cast<uint32_t>(a.D) * 2u;
            const uint32_t boff = 2u * (static_cast<uint32_t>(t) * nhs * static_cast<uint32_t>(a.D) + o);
            st16_device(buffer_rsrc(second ? a.out2 : a.out, bytes), boff, v);
        } else {
            st16_stream((second_lane ? out2 : out1) + o, v);
        }
    };

    // With QK-norm the angles are computed while the heads are in flight:
    // this lane's frequencies are loaded before the heads (vector loads
    // complete in order, so loaded after them they wait for every head), the
    // position right after them with a scalar load. Measured on MI355X for
    // Mistral-7B's Q and K at T = 4096: 17.8 us, against 18.6 us with both
    // loaded after the heads. Plain RoPE is faster with both loaded after the
    // heads, as vector loads (Q: 11.45 us, against 13.0 us with the angles
    // computed early, and 12.4-12.8 us with the stores held until every head
    // is in, or with one of the two round trips after the heads left): each
    // wave's two round trips between its last load and its first store keep
    // the grid's writes behind its reads. Small tensors (EARLY: up to 8 MiB,
    // one pass per wave) are bound by latency instead, and plain RoPE loads
    // the position (a vector load) and the frequencies ahead of the heads
    // too: Q at T = 64 2.19 us against 2.50, at T = 256 2.35 against 2.78.
    float f0 = 0.0f, f1 = 0.0f;
    int praw = 0;
    if (ROT && (QKNORM || EARLY)) {
        if (EARLY) praw = a.pos[t];
        f0 = a.inv_freq[lane < half ? lane : 0];
        if (half > kWave) f1 = a.inv_freq[lane + kWave < half ? lane + kWave : 0];
    }

    // Pass k of this wave is head pass g * HPL + k of the token: passes
    // [0, npass1) cover the first tensor, the rest the second. A pass (or a
    // lane) past the last head loads the first tensor's last head, and does
    // not store.
    u32x4 v1[HPL], v2[HPL];
    uint32_t off[HPL];  // element offsets within the token (unsigned: plain 32-bit address arithmetic)
    bool ok[HPL], sec[HPL];
#pragma unroll
    for (int k = 0; k < HPL; ++k) {
        const int pi = g * HPL + k;
        sec[k] = pi >= a.npass1;
        const int h = (sec[k] ? pi - a.npass1 : pi) * hpp + hl;
        ok[k] = h < (sec[k] ? a.nh2 : a.nh);
        const uint16_t* src = ok[k] && sec[k] ? in2 : in1;
        off[k] = static_cast<uint32_t>((ok[k] ? h : a.nh - 1) * a.D) | static_cast<uint32_t>(8 * j);  // 8 j < D
        v1[k] = ld16_stream(src + off[k]);
        if (STYLE == 0) v2[k] = ld16_stream(src + off[k] + half);
    }
    __builtin_amdgcn_sched_barrier(0);

    float s0 = 0.0f, c0 = 1.0f, s1 = 0.0f, c1 = 1.0f;
    auto angles = [&](int pos) {
        const float p = static_cast<float>(__builtin_amdgcn_readfirstlane(pos));
        sincosf(p * f0, &s0, &c0);
        if (half > kWave) sincosf(p * f1, &s1, &c1);
    };
    if (ROT && QKNORM) angles(a.pos[t]);
    if (EARLY) angles(praw);

    if (QKNORM) {
        // Per-head RMSNorm of each pass before it is rotated (weights of the
        // tensor the pass belongs to; the same vectors of the weight row for
        // every head).
        const uint16_t* wt1 = static_cast<const uint16_t*>(a.w1);
        const uint16_t* wt2 = a.nh2 > 0 ? static_cast<const uint16_t*>(a.w2) : wt1;
        u32x4 wa1 = ld16(wt1 + 8 * j), wa2 = ld16(wt2 + 8 * j), wb1 = wa1, wb2 = wa2;
        if (STYLE == 0) {
            wb1 = ld16(wt1 + half + 8 * j);
            wb2 = ld16(wt2 + half + 8 * j);
        }
#pragma unroll
        for (int k = 0; k < HPL; ++k) {
            if (STYLE == 0) {
                u32x4 xs[2] = {v1[k], v2[k]};
                const u32x4 ws[2] = {sec[k] ? wa2 : wa1, sec[k] ? wb2 : wb1};
                head_rmsnorm<T, 2>(xs, ws, lph, a.D, a.eps);
                v1[k] = xs[0];
                v2[k] = xs[1];
            } else {
                u32x4 xs[1] = {v1[k]};
                const u32x4 ws[1] = {sec[k] ? wa2 : wa1};
                head_rmsnorm<T, 1>(xs, ws, lph, a.D, a.eps);
                v1[k] = xs[0];
            }
        }
    }

    if (!ROT) {
        // Per-head RMSNorm alone (ng_per_head_rmsnorm): store the normalised heads.
#pragma unroll
        for (int k = 0; k < HPL; ++k) {
            if (!ok[k]) continue;
            store(sec[k], off[k], v1[k]);
            if (STYLE == 0) store(sec[k], off[k] + half, v2[k]);
        }
        return;
    }

    if (!QKNORM && !EARLY) {
        const float p = static_cast<float>(__builtin_amdgcn_readfirstlane(a.pos[t]));
        sincosf(p * a.inv_freq[lane < half ? lane : 0], &s0, &c0);
        if (half > kWave) sincosf(p * a.inv_freq[lane + kWave < half ? lane + kWave : 0], &s1, &c1);
    }

    constexpr int NP = STYLE == 0 ? 8 : 4;  // pairs per lane
    float c[NP], sn[NP];
#pragma unroll
    for (int e = 0; e < NP; ++e) {
        const int pi = NP * j + e;
        const int src = pi & (kWave - 1);
        const float cl = __shfl(c0, src, kWave), sl = __shfl(s0, src, kWave);
        if (half > kWave) {
            const float ch = __shfl(c1, src, kWave), sh = __shfl(s1, src, kWave);
            c[e] = pi < kWave ? cl : ch;
            sn[e] = pi < kWave ? sl : sh;
        } else {
            c[e] = cl;
            sn[e] = sl;
        }
    }

#pragma unroll
    for (int k = 0; k < HPL; ++k) {
        if (STYLE == 0) {
            float x1[8], x2[8], y1[8], y2[8];
            unpack8<T>(v1[k], x1);
            unpack8<T>(v2[k], x2);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                y1[e] = x1[e] * c[e] - x2[e] * sn[e];
                y2[e] = x1[e] * sn[e] + x2[e] * c[e];
            }
            if (ok[k]) {
                store(sec[k], off[k], pack8<T>(y1));
                store(sec[k], off[k] + half, pack8<T>(y2));
            }
        } else {
            float x[8], y[8];
            unpack8<T>(v1[k], x);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                y[2 * e] = x[2 * e] * c[e] - x[2 * e + 1] * sn[e];
                y[2 * e + 1] = x[2 * e] * sn[e] + x[2 * e + 1] * c[e];
            }
            if (ok[k]) store(sec[k], off[k], pack8<T>(y));
        }
    }
}

// Any head_dim and alignment: one thread per (token, head, pair).
template <typename T>
__global__ __launch_bounds__(kRopeThreads) void rope_scalar_kernel(RopeArgs a, int style) {
    const size_t npairs = static_cast<size_t>(a.T) * a.nh * a.half;
    const uint16_t* in = static_cast<const uint16_t*>(a.in);
    uint16_t* out = static_cast<uint16_t*>(a.out);
    const size_t stride = static_cast<size_t>(gridDim.x) * kRopeThreads;
    for (size_t p = static_cast<size_t>(blockIdx.x) * kRopeThreads + threadIdx.x; p < npairs; p += stride) {
        const int i = static_cast<int>(p % a.half);
        const size_t th = p / a.half;  // token * nh + head
        const int t = static_cast<int>(th / a.nh);
        const size_t base = th * a.D;
        const size_t i1 = style == 1 ? base + 2 * i : base + i;
        const size_t i2 = style == 1 ? base + 2 * i + 1 : base + i + a.half;
        float s, c;
        sincosf(static_cast<float>(a.pos[t]) * a.inv_freq[i], &s, &c);
        const float x1 = to_f32<T>(in[i1]), x2 = to_f32<T>(in[i2]);
        const float y1 = x1 * c - x2 * s;
        const float y2 = x1 * s + x2 * c;
        out[i1] = from_f32<T>(y1);
        out[i2] = from_f32<T>(y2);
    }
}

// inv_freq tables, cached per (theta bits, head_dim): 64 powf calls per miss.
void fill_inv_freq(float theta, int D, float* dst) {
    static std::mutex mu;
    static std::unordered_map<uint64_t, std::vector<float>> cache;
    const uint64_t key = (static_cast<uint64_t>(__builtin_bit_cast(uint32_t, theta)) << 32) |
                         static_cast<uint32_t>(D);
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it == cache.end()) {
        std::vector<float> v(D / 2);
        for (int i = 0; i < D / 2; ++i) {
            const float expo = (2.0f * static_cast<float>(i)) / static_cast<float>(D);
            v[i] = 1.0f / powf(theta, expo);
        }
        it = cache.emplace(key, std::move(v)).first;
    }
    for (int i = 0; i < D / 2; ++i) dst[i] = it->second[i];
}

static bool wave_rope_ok(int head_dim) { return head_dim == 64 || head_dim == 128 || head_dim == 256; }

// Launch rope_wave_kernel over one tensor [T, nh, D], or two tensors of the
// same tokens ([T, nh, D] and [T, nh2, D], nh2 > 0) that share positions.
template <typename T>
static int launch_rope_wave(const char* name, void* out, const void* in, void* out2, const void* in2,
                            const int* positions, int tokens, int nh, int nh2, int head_dim, int style,
                            const float* inv_freq, const void* w1 = nullptr, const void* w2 = nullptr,
                            float eps = 0.0f, bool rotate = true) {
    RopeWaveArgs w{};
    w.w1 = w1;
    w.w2 = w2;
    w.eps = eps;
    const bool qknorm = w1 != nullptr;
    w.out = out;
    w.in = in;
    w.out2 = out2;
    w.in2 = in2;
    w.pos = positions;
    w.T = tokens;
    w.nh = nh;
    w.nh2 = nh2;
    w.D = head_dim;
    // In-place updates of tensors up to 8 MiB: device-scope stores. Measured
    // on MI355X against non-temporal ones: K at Mistral-7B prefill (8 MiB)
    // 4.49 vs 4.66 us, at Mistral-Nemo (4 MiB) 3.16 vs 3.59 us, Q at decode
    // 2.48 vs 2.66 us; from 16 MiB on (Mistral-Nemo's Q) no faster.
    const long long bytes = 2ll * tokens * (nh + nh2) * head_dim;
    w.dev_store = out == in && (nh2 == 0 || out2 == in2) && bytes <= (8ll << 20);
    const int lph = style == 0 ? head_dim / 16 : head_dim / 8;
    w.lph_log2 = __builtin_ctz(static_cast<unsigned>(lph));
    const int hpp = kWave / lph;
    w.npass1 = (nh + hpp - 1) / hpp;
    const int npass = w.npass1 + (nh2 + hpp - 1) / hpp;
    // Waves per token: at most one per pass and at most 8 passes per wave;
    // below 4096 tokens, enough waves for 32 per CU (T = 2048, 32 heads:
    // 6.5 vs 6.9 us with one wave per token), from 4096 on one wave per
    // token (T = 4096: 11.0 vs 12.1 us with two).
    const long long want = (tokens >= 4096 ? 8ll : 32ll) * device_cu_count();
    int G = static_cast<int>((want + tokens - 1) / tokens);
    // From 8192 tokens on, one pass per wave (Llama-2-13B, 8192 x 40 heads:
    // 29.41 vs 29.59 us with the five passes of a token in one wave).
    if (tokens >= 8192) G = npass;
    if (G > npass) G = npass;
    if (G < (npass + 7) / 8) G = (npass + 7) / 8;
    if (G < 1) G = 1;
    const int hpl = (npass + G - 1) / G;
    G = (npass + hpl - 1) / hpl;
    w.G = G;
    w.div_G = make_fastdiv(static_cast<uint32_t>(G));
    if (inv_freq)
        for (int i = 0; i < head_dim / 2; ++i) w.inv_freq[i] = inv_freq[i];
    const long long waves = static_cast<long long>(tokens) * G;
    NG_REQUIRE(waves < (1ll << 31), "%s: tensor too large", name);
    // One-wave workgroups for one pass per wave from 8192 tokens on and for
    // tensors up to 1 MiB (decode), four-wave ones otherwise. Measured on
    // MI355X, four against one wave per workgroup: Llama-2-13B's Q (8192 x 40
    // heads) 29.30 vs 28.67 us, Q at T = 64 2.20 vs 2.11 us, K at T = 64 2.22
    // vs 2.10 us; Mistral-7B's K at T = 4096 (8 MiB) 4.54 vs 4.85 us,
    // Mistral-Nemo's K (4 MiB) 2.63 vs 2.98 us, Q and K in one launch at
    // T = 4096 14.47 vs 14.85 us, Q at T = 2048 6.63 vs 6.72 us.
    const bool small = rotate && !qknorm && bytes <= (8ll << 20);
    const int wpb = hpl == 1 && (tokens >= 8192 || (small && bytes <= (1ll << 20))) ? 1 : kRopeThreads / kWave;
    const unsigned blocks = static_cast<unsigned>((waves + wpb - 1) / wpb);
    auto go = [&](auto kern) { kern<<<dim3(blocks), dim3(wpb * kWave), 0, stream()>>>(w); };
#define NG_ROPE_WAVE(HPL)                                                                   \
    case HPL:                                                                               \
        if (!rotate) {                                                                      \
            go(rope_wave_kernel<T, 0, HPL, true, false>);                                   \
        } else if (qknorm) {                                                                \
            if (style == 0) go(rope_wave_kernel<T, 0, HPL, true>);                          \
            else go(rope_wave_kernel<T, 1, HPL, true>);                                     \
        } else {                                                                            \
            if (style == 0) go(rope_wave_kernel<T, 0, HPL, false>);                         \
            else go(rope_wave_kernel<T, 1, HPL, false>);                                    \
        }                                                                                   \
        break;
    // Up to 8 MiB with one pass per wave, plain RoPE takes the variant that
    // loads the position and the frequencies ahead of the heads.
    if (hpl == 1 && small) {
        if (style == 0) go(rope_wave_kernel<T, 0, 1, false, true, true>);
        else go(rope_wave_kernel<T, 1, 1, false, true, true>);
        return 0;
    }
    switch (hpl) {
        NG_ROPE_WAVE(1) NG_ROPE_WAVE(2) NG_ROPE_WAVE(3) NG_ROPE_WAVE(4)
        NG_ROPE_WAVE(5) NG_ROPE_WAVE(6) NG_ROPE_WAVE(7) NG_ROPE_WAVE(8)
        default: NG_REQUIRE(false, "%s: internal: %d passes per wave", name, hpl);
    }
#undef NG_ROPE_WAVE
    return 0;
}

template <typename T>
static int launch_rope(const char* name, void* output, const void* input, const int* positions,
                       int batch_size, int seq_len, int num_heads, int head_dim, int style, float theta) {
    NG_REQUIRE(output && input && positions, "%s: null pointer", name);
    NG_REQUIRE(batch_size > 0 && seq_len > 0 && num_heads > 0, "%s: batch=%d seq=%d heads=%d must be > 0",
               name, batch_size, seq_len, num_heads);
    NG_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 2 * kRopeMaxHalf,
               "%s: head_dim=%d must be even and in [2, %d]", name, head_dim, 2 * kRopeMaxHalf);
    // As in the reference (kernels.cu:469), every style other than 1 pairs split-half.
    style = style == 1 ? 1 : 0;
    const long long T64 = static_cast<long long>(batch_size) * seq_len;
    NG_REQUIRE(T64 * num_heads * head_dim < (1ll << 31), "%s: tensor too large", name);

    RopeArgs a{};
    a.out = output;
    a.in = input;
    a.pos = positions;
    a.T = static_cast<int>(T64);
    a.nh = num_heads;
    a.D = head_dim;
    a.half = head_dim / 2;
    fill_inv_freq(theta, head_dim, a.inv_freq);

    const bool aligned = aligned16(output) && aligned16(input);
    const bool vec = aligned && ((style == 0 && head_dim % 16 == 0) || (style == 1 && head_dim % 8 == 0));
    if (aligned && wave_rope_ok(head_dim)) {
        const int rc = launch_rope_wave<T>(name, output, input, output, input, positions, a.T, num_heads, 0,
                                           head_dim, style, a.inv_freq);
        if (rc != 0) return rc;
    } else if (vec) {
        const int uph = style == 0 ? head_dim / 16 : head_dim / 8;
        a.upt = num_heads * uph;
        const long long units = static_cast<long long>(a.T) * a.upt;
        NG_REQUIRE(units < (1ll << 31), "%s: tensor too large", name);
        a.units = static_cast<int>(units);
        a.div_upt = make_fastdiv(static_cast<uint32_t>(a.upt));
        a.div_uph = make_fastdiv(static_cast<uint32_t>(uph));
        a.div_half = make_fastdiv(static_cast<uint32_t>(a.half));
        // Units per thread: as many as keep at least two workgroups per CU.
        const long long min_blocks = 2ll * device_cu_count();
        int U = 4;
        while (U > 1 && (units + kRopeThreads * U - 1) / (kRopeThreads * U) < min_blocks) U >>= 1;
        const int per_block = kRopeThreads * U;
        const unsigned blocks = static_cast<unsigned>((units + per_block - 1) / per_block);
        const int max_tok = (per_block + a.upt - 1) / a.upt + 1;
        const size_t lds = static_cast<size_t>(max_tok) * a.half * sizeof(float2);
        NG_REQUIRE(lds <= 64 * 1024, "%s: head_dim=%d needs %zu bytes of LDS", name, head_dim, lds);
        auto go = [&](auto kern) { kern<<<dim3(blocks), dim3(kRopeThreads), lds, stream()>>>(a); };
        if (style == 0) {
            if (U == 4) go(rope_vec_kernel<T, 0, 4>);
            else if (U == 2) go(rope_vec_kernel<T, 0, 2>);
            else go(rope_vec_kernel<T, 0, 1>);
        } else {
            if (U == 4) go(rope_vec_kernel<T, 1, 4>);
            else if (U == 2) go(rope_vec_kernel<T, 1, 2>);
            else go(rope_vec_kernel<T, 1, 1>);
        }
    } else {
        const size_t npairs = static_cast<size_t>(a.T) * num_heads * a.half;
        size_t blocks = (npairs + kRopeThreads - 1) / kRopeThreads;
        if (blocks > 65536) blocks = 65536;
        rope_scalar_kernel<T><<<dim3(static_cast<unsigned>(blocks)), dim3(kRopeThreads), 0, stream()>>>(a, style);
    }
    NG_CHECK_LAUNCH(name);
    return 0;
}

}  // namespace ng

using namespace ng;

extern "C" int cuda_rope_with_theta(void* output, const void* input, const int* positions, int batch_size,
                                    int seq_len, int num_heads, int head_dim, int rope_style, float rope_theta) {
    return launch_rope<f16>("cuda_rope_with_theta", output, input, positions, batch_size, seq_len, num_heads,
                            head_dim, rope_style, rope_theta);
}

extern "C" int cuda_rope_styled(void* output, const void* input, const int* positions, int batch_size,
                                int seq_len, int num_heads, int head_dim, int rope_style) {
    return launch_rope<f16>("cuda_rope_styled", output, input, positions, batch_size, seq_len, num_heads,
                            head_dim, rope_style, 10000.0f);
}

extern "C" int cuda_rope(void* output, const void* input, const int* positions, int batch_size, int seq_len,
                         int num_heads, int head_dim) {
    return launch_rope<f16>("cuda_rope", output, input, positions, batch_size, seq_len, num_heads, head_dim,
                            0, 10000.0f);
}

extern "C" int cuda_bf16_rope_with_theta(void* output, const void* input, const int* positions, int batch_size,
                                         int seq_len, int num_heads, int head_dim, int rope_style,
                                         float rope_theta) {
    return launch_rope<bf16>("cuda_bf16_rope_with_theta", output, input, positions, batch_size, seq_len,
                             num_heads, head_dim, rope_style, rope_theta);
}

// Q and K of the same tokens in one launch (the pair of calls at
// gpu/engine/layer.cu:1016,1018, fused): each token's angles are evaluated
// once for both tensors. Falls back to two launches for head_dim outside
// {64, 128, 256} or unaligned buffers.
template <typename T>
static int launch_rope_qk(const char* name, void* q_out, const void* q_in, void* k_out, const void* k_in,
                          const int* positions, int batch_size, int seq_len, int num_q_heads, int num_kv_heads,
                          int head_dim, int style, float theta,
                          int (*single)(void*, const void*, const int*, int, int, int, int, int, float)) {
    NG_REQUIRE(q_out && q_in && k_out && k_in && positions, "%s: null pointer", name);
    NG_REQUIRE(batch_size > 0 && seq_len > 0 && num_q_heads > 0 && num_kv_heads > 0,
               "%s: batch=%d seq=%d q_heads=%d kv_heads=%d must be > 0", name, batch_size, seq_len, num_q_heads,
               num_kv_heads);
    NG_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 2 * kRopeMaxHalf,
               "%s: head_dim=%d must be even and in [2, %d]", name, head_dim, 2 * kRopeMaxHalf);
    style = style == 1 ? 1 : 0;
    const long long T64 = static_cast<long long>(batch_size) * seq_len;
    NG_REQUIRE(T64 * num_q_heads * head_dim < (1ll << 31) && T64 * num_kv_heads * head_dim < (1ll << 31),
               "%s: tensor too large", name);
    const bool aligned = aligned16(q_out) && aligned16(q_in) && aligned16(k_out) && aligned16(k_in);
    if (!(aligned && wave_rope_ok(head_dim))) {
        const int rc = single(q_out, q_in, positions, batch_size, seq_len, num_q_heads, head_dim, style, theta);
        if (rc != 0) return rc;
        return single(k_out, k_in, positions, batch_size, seq_len, num_kv_heads, head_dim, style, theta);
    }
    float inv[kRopeMaxHalf];
    fill_inv_freq(theta, head_dim, inv);
    const int rc = launch_rope_wave<T>(name, q_out, q_in, k_out, k_in, positions, static_cast<int>(T64), num_q_heads,
                                       num_kv_heads, head_dim, style, inv);
    if (rc != 0) return rc;
    NG_CHECK_LAUNCH(name);
    return 0;
}

extern "C" int ng_rope_qk_with_theta(void* q_out, const void* q_in, void* k_out, const void* k_in,
                                     const int* positions, int batch_size, int seq_len, int num_q_heads,
                                     int num_kv_heads, int head_dim, int rope_style, float rope_theta) {
    return launch_rope_qk<f16>("ng_rope_qk_with_theta", q_out, q_in, k_out, k_in, positions, batch_size, seq_len,
                               num_q_heads, num_kv_heads, head_dim, rope_style, rope_theta, cuda_rope_with_theta);
}

extern "C" int ng_bf16_rope_qk_with_theta(void* q_out, const void* q_in, void* k_out, const void* k_in,
                                          const int* positions, int batch_size, int seq_len, int num_q_heads,
                                          int num_kv_heads, int head_dim, int rope_style, float rope_theta) {
    return launch_rope_qk<bf16>("ng_bf16_rope_qk_with_theta", q_out, q_in, k_out, k_in, positions, batch_size,
                                seq_len, num_q_heads, num_kv_heads, head_dim, rope_style, rope_theta,
                                cuda_bf16_rope_with_theta);
}

// Per-head RMSNorm of Q and K followed by RoPE, in one launch (the QK
// LayerNorm of gpu/engine/layer.cu:998-1013 and the RoPE pair of :1016-1018).
// The normalisation is exactly ng_per_head_rmsnorm's, rounded to the element
// type, and the rotation is cuda_rope_with_theta's applied to that result.
// head_dim outside {64, 128, 256} or unaligned buffers take the two steps as
// separate launches.
template <typename T>
static int launch_qk_norm_rope(const char* name, void* q_out, const void* q_in, void* k_out, const void* k_in,
                               const void* q_weight, const void* k_weight, const int* positions, int batch_size,
                               int seq_len, int num_q_heads, int num_kv_heads, int head_dim, float eps, int style,
                               float theta,
                               int (*norm)(void*, const void*, const void*, int, int, int, float),
                               int (*rope)(void*, const void*, const int*, int, int, int, int, int, float)) {
    NG_REQUIRE(q_out && q_in && k_out && k_in && q_weight && k_weight && positions, "%s: null pointer", name);
    NG_REQUIRE(batch_size > 0 && seq_len > 0 && num_q_heads > 0 && num_kv_heads > 0,
               "%s: batch=%d seq=%d q_heads=%d kv_heads=%d must be > 0", name, batch_size, seq_len, num_q_heads,
               num_kv_heads);
    NG_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 2 * kRopeMaxHalf,
               "%s: head_dim=%d must be even and in [2, %d]", name, head_dim, 2 * kRopeMaxHalf);
    style = style == 1 ? 1 : 0;
    const long long T64 = static_cast<long long>(batch_size) * seq_len;
    NG_REQUIRE(T64 * num_q_heads * head_dim < (1ll << 31) && T64 * num_kv_heads * head_dim < (1ll << 31),
               "%s: tensor too large", name);
    const bool aligned = aligned16(q_out) && aligned16(q_in) && aligned16(k_out) && aligned16(k_in) &&
                         aligned16(q_weight) && aligned16(k_weight);
    if (!(aligned && wave_rope_ok(head_dim))) {
        const int T32 = static_cast<int>(T64);
        int rc = norm(q_out, q_in, q_weight, T32, num_q_heads, head_dim, eps);
        if (rc == 0) rc = norm(k_out, k_in, k_weight, T32, num_kv_heads, head_dim, eps);
        if (rc == 0) rc = rope(q_out, q_out, positions, batch_size, seq_len, num_q_heads, head_dim, style, theta);
        if (rc == 0) rc = rope(k_out, k_out, positions, batch_size, seq_len, num_kv_heads, head_dim, style, theta);
        return rc;
    }
    float inv[kRopeMaxHalf];
    fill_inv_freq(theta, head_dim, inv);
    const int rc = launch_rope_wave<T>(name, q_out, q_in, k_out, k_in, positions, static_cast<int>(T64), num_q_heads,
                                       num_kv_heads, head_dim, style, inv, q_weight, k_weight, eps);
    if (rc != 0) return rc;
    NG_CHECK_LAUNCH(name);
    return 0;
}

extern "C" int ng_qk_rmsnorm_rope_with_theta(void* q_out, const void* q_in, void* k_out, const void* k_in,
                                             const void* q_norm_weight, const void* k_norm_weight,
                                             const int* positions, int batch_size, int seq_len, int num_q_heads,
                                             int num_kv_heads, int head_dim, float eps, int rope_style,
                                             float rope_theta) {
    return launch_qk_norm_rope<f16>("ng_qk_rmsnorm_rope_with_theta", q_out, q_in, k_out, k_in, q_norm_weight,
                                    k_norm_weight, positions, batch_size, seq_len, num_q_heads, num_kv_heads,
                                    head_dim, eps, rope_style, rope_theta, ng_per_head_rmsnorm,
                                    cuda_rope_with_theta);
}

extern "C" int ng_bf16_qk_rmsnorm_rope_with_theta(void* q_out, const void* q_in, void* k_out, const void* k_in,
                                                  const void* q_norm_weight, const void* k_norm_weight,
                                                  const int* positions, int batch_size, int seq_len,
                                                  int num_q_heads, int num_kv_heads, int head_dim, float eps,
                                                  int rope_style, float rope_theta) {
    return launch_qk_norm_rope<bf16>("ng_bf16_qk_rmsnorm_rope_with_theta", q_out, q_in, k_out, k_in, q_norm_weight,
                                     k_norm_weight, positions, batch_size, seq_len, num_q_heads, num_kv_heads,
                                     head_dim, eps, rope_style, rope_theta, ng_bf16_per_head_rmsnorm,
                                     cuda_bf16_rope_with_theta);
}

// Per-head RMSNorm alone: the wave kernel without the rotation for head_dim
// 64, 128 or 256 (a head is spread over head_dim / 16 lanes, every lane busy);
// other head_dim or unaligned buffers use the row kernel over tokens * heads
// rows of head_dim.
template <typename T>
static int launch_per_head_rmsnorm(const char* name, void* output, const void* input, const void* weight,
                                   int num_tokens, int num_heads, int head_dim, float eps) {
    NG_REQUIRE(output && input && weight, "%s: null pointer", name);
    NG_REQUIRE(num_tokens > 0 && num_heads > 0 && head_dim > 0, "%s: tokens=%d heads=%d head_dim=%d must be > 0",
               name, num_tokens, num_heads, head_dim);
    NG_REQUIRE(static_cast<long long>(num_tokens) * num_heads * head_dim < (1ll << 31), "%s: tensor too large",
               name);
    if (aligned16(output) && aligned16(input) && aligned16(weight) && wave_rope_ok(head_dim)) {
        const int rc = launch_rope_wave<T>(name, output, input, output, input, nullptr, num_tokens, num_heads, 0,
                                           head_dim, 0, nullptr, weight, weight, eps, false);
        if (rc != 0) return rc;
        NG_CHECK_LAUNCH(name);
        return 0;
    }
    return rows_rmsnorm<T>(name, output, input, weight, num_tokens * num_heads, head_dim, eps);
}

extern "C" int ng_per_head_rmsnorm(void* output, const void* input, const void* weight, int num_tokens,
                                   int num_heads, int head_dim, float eps) {
    return launch_per_head_rmsnorm<f16>("ng_per_head_rmsnorm", output, input, weight, num_tokens, num_heads,
                                        head_dim, eps);
}

extern "C" int ng_bf16_per_head_rmsnorm(void* output, const void* input, const void* weight, int num_tokens,
                                        int num_heads, int head_dim, float eps) {
    return launch_per_head_rmsnorm<bf16>("ng_bf16_per_head_rmsnorm", output, input, weight, num_tokens, num_heads,
                                         head_dim, eps);
}
