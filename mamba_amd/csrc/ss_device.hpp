// Device-side helpers shared by the forward and backward selective-scan
// kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <utility>

namespace ss {

// ---------------------------------------------------------------- tiling --
// A wave is 4 rows of 16 lanes.  Row j holds one channel; lane r of the row
// holds state n = 16 * s + r of state group s.  Time is walked sequentially
// in tiles of kT = 16 steps: at the start of a tile, lane r also owns the
// per-step inputs of step t0 + r (delta, u, z, dout), which the other lanes
// of the row read through DPP row broadcasts.
constexpr int kT = 16;            // steps per tile == lanes per row
constexpr int kRows = 4;          // channels per wave
constexpr int kWaves = 4;         // waves per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kChPerWG = kRows * kWaves;
constexpr int kChunk = 32;        // steps per checkpoint of the state h
constexpr int kMaxSPL = 16;       // state groups: dstate <= 16 * kMaxSPL = 256
constexpr float kLog2e = 1.4426950408889634f;

// Scratch layout of the in-row transposed sum: per row, 16 lanes x 16
// values with a stride of 20 floats (keeps float4 alignment and spreads
// banks), plus 16 floats of padding so the four rows start on different
// banks.
constexpr int kTrStride = 20;
constexpr int kTrRow = kT * kTrStride + 16;       // 336 floats
constexpr int kTrWave = kRows * kTrRow;           // 1344 floats

// ------------------------------------------------------------ data types --
struct bf16_t { uint16_t bits; };

template <typename T> struct io;
template <> struct io<float> {
    static __device__ __forceinline__ float load(const float* p) { return *p; }
    static __device__ __forceinline__ void store(float* p, float v) { *p = v; }
};
template <> struct io<bf16_t> {
    static __device__ __forceinline__ float load(const bf16_t* p) {
        return __uint_as_float(uint32_t(p->bits) << 16);
    }
    static __device__ __forceinline__ uint16_t round(float v) {
        uint32_t u = __float_as_uint(v);
        if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);  // quiet NaN
        u += 0x7fffu + ((u >> 16) & 1u);                                           // RNE
        return uint16_t(u >> 16);
    }
    static __device__ __forceinline__ void store(bf16_t* p, float v) { p->bits = round(v); }
};
template <> struct io<_Float16> {
    static __device__ __forceinline__ float load(const _Float16* p) { return float(*p); }
    static __device__ __forceinline__ void store(_Float16* p, float v) { *p = _Float16(v); }
};

// Loads 16 consecutive elements p[0..15] as float; positions >= nvalid read
// as 0.  `vec` says p is 16-byte aligned (then full tiles use 16-byte loads).
template <typename T>
__device__ __forceinline__ void load16(const T* __restrict__ p, int nvalid, bool vec, float (&o)[16]) {
    if (nvalid >= 16 && vec) {
        if constexpr (sizeof(T) == 4) {
            const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float4 v = q[i];
                o[4 * i] = v.x; o[4 * i + 1] = v.y; o[4 * i + 2] = v.z; o[4 * i + 3] = v.w;
            }
        } else {
            const uint4* q = reinterpret_cast<const uint4*>(p);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                uint4 v = q[i];
                uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if constexpr (sizeof(T) == 2 && __is_same(T, bf16_t)) {
                        o[8 * i + 2 * k] = __uint_as_float(w[k] << 16);
                        o[8 * i + 2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
                    } else {
                        o[8 * i + 2 * k] = float(__builtin_bit_cast(_Float16, uint16_t(w[k] & 0xffffu)));
                        o[8 * i + 2 * k + 1] = float(__builtin_bit_cast(_Float16, uint16_t(w[k] >> 16)));
                    }
                }
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) o[i] = i < nvalid ? io<T>::load(p + i) : 0.f;
    }
}

// ------------------------------------------------------- cross-lane ops --
// Value of lane K of this lane's 16-lane row (DPP row_newbcast); folds into
// the consuming VALU instruction as a DPP source modifier.
template <int K>
__device__ __forceinline__ float row_bcast(float v) {
    static_assert(K >= 0 && K < 16, "row lane");
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                 0x150 + K, 0xf, 0xf, false));
}

// Sum over the 16 lanes of a row, result in every lane of the row.
__device__ __forceinline__ float row_allsum(float v) {
    // row_shr-free butterfly: xor 1, 2 via quad_perm; xor 4, 8 via row_ror
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false)); // quad_perm [1,0,3,2]
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xf, 0xf, false)); // quad_perm [2,3,0,1]
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false)); // row_ror:4
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false)); // row_ror:8
    return v;
}

// In-row transposed sum: lane r of row j passes v[0..15]; the result in lane
// r is sum over the row's lanes r' of v_{r'}[r].  `wbuf` is this wave's
// private scratch of kTrWave floats.  Only lanes of the calling wave touch
// it and a wave executes its LDS operations in order, so no barrier is
// needed; the compiler cannot reorder the accesses because their offsets
// depend on the lane index.
__device__ __forceinline__ float row_transpose_sum(float* wbuf, const float (&v)[16], int j, int r) {
    float* wp = wbuf + j * kTrRow + r * kTrStride;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        *reinterpret_cast<float4*>(wp + 4 * i) = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    const float* rp = wbuf + j * kTrRow + r;
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int k = 0; k < 16; k += 2) {
        s0 += rp[k * kTrStride];
        s1 += rp[(k + 1) * kTrStride];
    }
    return s0 + s1;
}

// ------------------------------------------------------------ unrolling --
template <typename F, int... Ks>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Ks...>) {
    (f(std::integral_constant<int, Ks>{}), ...);
}
// Calls f(integral_constant<int, k>) for k = 0 .. N-1 in order.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// ----------------------------------------------------------------- math --
__device__ __forceinline__ float softplus20(float x) {
    // log1p(exp(x)) below the threshold 20, x above (forward_kernel.cu:217-221)
    return x <= 20.f ? log1pf(__expf(x)) : x;
}
__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + __expf(-x)); }

}  // namespace ss
