// RMSNorm with an optional residual add, forward and backward, on gfx950.
//
// The reference normalises in PyTorch (modules/rms_norm.py:19,29-31) and adds
// the residual after each block (models/causal_lm.py:31-35):
//
//   s    = x + residual                       (rounded to the I/O type)
//   rstd = rsqrt(mean(s^2) + eps)             (fp32)
//   out  = (s * rstd) * (1 + weight)          (fp32, rounded to the I/O type)
//
// Backward, with g = dout * (1 + weight):
//
//   ds       = rstd * g - s * rstd^3 * sum(g * s) / dim  (+ dresidual_out)
//   dweight  = sum over rows of dout * s * rstd
//
// Layout: rows of `dim` elements with unit column stride.  One wave owns a
// row at a time; its 64 lanes read consecutive 16-byte vectors, so every
// load and store instruction moves 1 KiB of contiguous row.  A row is held
// in registers in segments of a few vectors per lane (4 KiB of row per
// forward segment; 2 KiB per backward segment, which also holds dout).  The
// sum of squares needs the whole row, so a row longer than one segment is
// read a second time for the output pass (from L2: the wave has just read
// it).  Outputs must not overlap inputs.  Rows whose size or alignment does not allow 16-byte
// vectors take the same code with one element per lane per slot.
//
// The forward is HBM-bound: it reads x (and the residual) and writes out
// (and the residual sum) once.  The backward reads s, dout (and the residual
// gradient) and writes dx once; its dweight column sums are accumulated per
// workgroup in LDS, written as one fp32 row per workgroup, and summed by a
// second kernel in a fixed order, so dweight is the same from run to run.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/mamba_ss.h"
#include "ss_device.hpp"
#include "ss_kernels.hpp"

namespace ss {

namespace {

constexpr int kNSF = 4;              // forward: vectors per lane per segment
constexpr int kNSB = 2;              // backward: vectors per lane per segment (it holds s and dout)
constexpr int kFwdWaves = 4;         // forward: rows per workgroup
constexpr int64_t kRmsNormPreRows = 1024;   // forward: at most this many rows preload the weight
constexpr int kBwdWaves = 8;         // backward: waves per workgroup
constexpr int kRedWaves = 16;        // dweight reduction: waves per workgroup

struct NormParams {
    int64_t rows, dim;
    int64_t x_rs, r_rs, o_rs, ro_rs;         // forward row strides (elements)
    int64_t s_rs, dy_rs, dr_rs, dx_rs;       // backward row strides
    const void* x; const void* r; const void* w;
    void* out; void* rout; float* rstd;
    const void* s; const void* dy; const void* dr; void* dx;
    float* part;                             // backward: (gridDim.x, dim) fp32
    float eps;
};

// VE consecutive elements of T as float, and back (VE * sizeof(T) is 16
// bytes on the vector path, VE = 1 otherwise)
// The VE elements of a 16-byte vector of T, as float.
template <typename T, int VE>
__device__ __forceinline__ void vunpack(const uint4& v, float (&o)[VE]) {
    if constexpr (sizeof(T) == 4) {
        static_assert(VE == 4, "16-byte vectors");
        o[0] = __uint_as_float(v.x); o[1] = __uint_as_float(v.y);
        o[2] = __uint_as_float(v.z); o[3] = __uint_as_float(v.w);
    } else {
        static_assert(VE == 8, "16-byte vectors");
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if constexpr (__is_same(T, bf16_t)) {
                o[2 * k] = __uint_as_float(w[k] << 16);
                o[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
            } else {
                o[2 * k] = float(__builtin_bit_cast(_Float16, uint16_t(w[k] & 0xffffu)));
                o[2 * k + 1] = float(__builtin_bit_cast(_Float16, uint16_t(w[k] >> 16)));
            }
        }
    }
}

template <typename T, int VE>
__device__ __forceinline__ void vload(const T* p, float (&o)[VE]) {
    if constexpr (VE == 1) {
        o[0] = io<T>::load(p);
    } else {
        vunpack<T, VE>(*reinterpret_cast<const uint4*>(p), o);
    }
}

template <typename T, int VE>
__device__ __forceinline__ void vstore(T* p, const float (&v)[VE]) {
    if constexpr (VE == 1) {
        io<T>::store(p, v[0]);
    } else if constexpr (sizeof(T) == 4) {
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if constexpr (__is_same(T, bf16_t)) {
                w[k] = io<bf16_t>::pack2(v[2 * k], v[2 * k + 1]);
            } else {
                w[k] = uint32_t(__builtin_bit_cast(uint16_t, _Float16(v[2 * k]))) |
                       (uint32_t(__builtin_bit_cast(uint16_t, _Float16(v[2 * k + 1]))) << 16);
            }
        }
        *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// v rounded to T and back to float
template <typename T>
__device__ __forceinline__ float round_to(float v) {
    if constexpr (sizeof(T) == 4) {
        return v;
    } else if constexpr (__is_same(T, bf16_t)) {
        return __uint_as_float(uint32_t(io<bf16_t>::round(v)) << 16);
    } else {
        return float(_Float16(v));
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// 1 + weight for the VE elements of vector vi
template <typename TW, int VE>
__device__ __forceinline__ void load_w1(const TW* w, int64_t vi, float (&o)[VE]) {
#pragma unroll
    for (int e = 0; e < VE; ++e) o[e] = 1.f + io<TW>::load(w + vi * VE + e);
}

// kPre: a row of one segment (dim <= 64 * kNSF * VE) requests its
// 1 + weight before the sum, so it waits for memory once; taken for few rows
// (decode steps), where the launch is latency-bound.  Many rows keep the
// lower register count (bf16 rows at 32768 x 768: 30.7 us
// without, 32.7 us with, from the lower occupancy).
template <typename T, typename TW, int VE, bool kPre>
__global__ __launch_bounds__(64 * kFwdWaves) void rmsnorm_fwd_kernel(const NormParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= p.rows) return;                          // no barrier in this kernel
    const T* xr = static_cast<const T*>(p.x) + row * p.x_rs;
    const T* rr = p.r ? static_cast<const T*>(p.r) + row * p.r_rs : nullptr;
    T* rout = p.rout ? static_cast<T*>(p.rout) + row * p.ro_rs : nullptr;
    T* outr = static_cast<T*>(p.out) + row * p.o_rs;
    const TW* w = static_cast<const TW*>(p.w);
    const int64_t nvec = p.dim / VE;
    const int nseg = int((nvec + 64 * kNSF - 1) / (64 * kNSF));

    float s[kNSF][VE];
    // s for segment g into registers; returns this lane's sum of squares
    auto load_seg = [&](int g, bool write_rout) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < kNSF; ++k) {
            const int64_t vi = (int64_t(g) * kNSF + k) * 64 + lane;
            if (vi < nvec) {
                vload<T, VE>(xr + vi * VE, s[k]);
                if (rr) {
                    float rv[VE];
                    vload<T, VE>(rr + vi * VE, rv);
#pragma unroll
                    for (int e = 0; e < VE; ++e) s[k][e] = round_to<T>(s[k][e] + rv[e]);
                    if (write_rout) vstore<T, VE>(rout + vi * VE, s[k]);
                }
#pragma unroll
                for (int e = 0; e < VE; ++e) acc = __builtin_fmaf(s[k][e], s[k][e], acc);
            }
        }
        return acc;
    };

    float w1p[kNSF][VE];
    const bool one = kPre && nseg == 1;
    if (one) {
#pragma unroll
        for (int k = 0; k < kNSF; ++k) {
            const int64_t vi = int64_t(k) * 64 + lane;
            if (vi < nvec) load_w1<TW, VE>(w, vi, w1p[k]);
        }
    }
    float ss = 0.f;
    for (int g = 0; g < nseg; ++g) ss += load_seg(g, rout != nullptr);
    ss = wave_sum(ss);
    const float rstd = rsqrtf(ss / float(p.dim) + p.eps);
    if (p.rstd && lane == 0) p.rstd[row] = rstd;

    // output pass, last segment first: it is still in registers
    for (int g = nseg - 1; g >= 0; --g) {
        if (g != nseg - 1) (void)load_seg(g, false);
#pragma unroll
        for (int k = 0; k < kNSF; ++k) {
            const int64_t vi = (int64_t(g) * kNSF + k) * 64 + lane;
            if (vi < nvec) {
                float w1[VE], o[VE];
                if (one) {
#pragma unroll
                    for (int e = 0; e < VE; ++e) w1[e] = w1p[k][e];
                } else {
                    load_w1<TW, VE>(w, vi, w1);
                }
#pragma unroll
                for (int e = 0; e < VE; ++e) o[e] = (s[k][e] * rstd) * w1[e];
                vstore<T, VE>(outr + vi * VE, o);
            }
        }
    }
}

// Backward rows that fit one register segment (the whole row is in the
// lane's slots): the wave keeps 1 + weight and its dweight column sums in
// registers for all of its rows; each row is one round trip (s, dout,
// dresidual_out and rstd are all requested before any is used) and stays
// packed in registers, unpacked where it is used.
template <typename T, typename TW, int VE>
__device__ __forceinline__ void bwd_rows_resident(const NormParams& p, float* s_dw, int lane, int64_t nvec,
                                                  int64_t row0, int64_t rstride) {
    const TW* w = static_cast<const TW*>(p.w);
    const float inv_dim = 1.f / float(p.dim);
    float w1[kNSB][VE], acc[kNSB][VE];
#pragma unroll
    for (int k = 0; k < kNSB; ++k) {
        const int64_t vi = int64_t(k) * 64 + lane;
#pragma unroll
        for (int e = 0; e < VE; ++e) {
            w1[k][e] = vi < nvec ? 1.f + io<TW>::load(w + vi * VE + e) : 0.f;
            acc[k][e] = 0.f;
        }
    }
    for (int64_t row = row0; row < p.rows; row += rstride) {
        const T* sr = static_cast<const T*>(p.s) + row * p.s_rs;
        const T* dyr = static_cast<const T*>(p.dy) + row * p.dy_rs;
        const T* drr = static_cast<const T*>(p.dr) + row * p.dr_rs;
        uint4 cs[kNSB], cd[kNSB], cr[kNSB];
#pragma unroll
        for (int k = 0; k < kNSB; ++k) {
            const int64_t vi = int64_t(k) * 64 + lane;
            cs[k] = cd[k] = cr[k] = make_uint4(0u, 0u, 0u, 0u);
            if (vi < nvec) {
                cs[k] = *reinterpret_cast<const uint4*>(sr + vi * VE);
                cd[k] = *reinterpret_cast<const uint4*>(dyr + vi * VE);
                if (p.dr) cr[k] = *reinterpret_cast<const uint4*>(drr + vi * VE);
            }
        }
        const float rstd = p.rstd[row];

        float dot = 0.f;
#pragma unroll
        for (int k = 0; k < kNSB; ++k) {
            float sv[VE], dv[VE];
            vunpack<T, VE>(cs[k], sv);
            vunpack<T, VE>(cd[k], dv);
#pragma unroll
            for (int e = 0; e < VE; ++e) dot = __builtin_fmaf(dv[e] * w1[k][e], sv[e], dot);
        }
        dot = wave_sum(dot);                            // slots past the row end hold zeros
        const float c = rstd * rstd * rstd * dot * inv_dim;
        T* dxr = static_cast<T*>(p.dx) + row * p.dx_rs;
#pragma unroll
        for (int k = 0; k < kNSB; ++k) {
            const int64_t vi = int64_t(k) * 64 + lane;
            if (vi < nvec) {
                float sv[VE], dv[VE], o[VE];
                vunpack<T, VE>(cs[k], sv);
                vunpack<T, VE>(cd[k], dv);
#pragma unroll
                for (int e = 0; e < VE; ++e) {
                    o[e] = rstd * (dv[e] * w1[k][e]) - c * sv[e];
                    acc[k][e] = __builtin_fmaf(dv[e], sv[e] * rstd, acc[k][e]);
                }
                if (p.dr) {
                    float rv[VE];
                    vunpack<T, VE>(cr[k], rv);
#pragma unroll
                    for (int e = 0; e < VE; ++e) o[e] += rv[e];
                }
                vstore<T, VE>(dxr + vi * VE, o);
            }
        }
    }
    // this wave's column sums into its own LDS region (plain stores: no
    // other wave writes there)
#pragma unroll
    for (int k = 0; k < kNSB; ++k) {
        const int64_t vi = int64_t(k) * 64 + lane;
        if (vi < nvec) {
#pragma unroll
            for (int e = 0; e < VE; ++e) s_dw[e * nvec + vi] = acc[k][e];
        }
    }
}

// Backward rows of any length: segments of kNSB vectors per lane, the
// second pass re-reading a row longer than one segment from L2, dweight
// column sums added into the wave's LDS region per row (a wave's own LDS
// operations execute in order, so each sum is formed in row order).
template <typename T, typename TW, int VE>
__device__ __forceinline__ void bwd_rows_general(const NormParams& p, float* s_dw, int lane, int64_t nvec,
                                                 int64_t row0, int64_t rstride) {
    const TW* w = static_cast<const TW*>(p.w);
    const int nseg = int((nvec + 64 * kNSB - 1) / (64 * kNSB));
    const float inv_dim = 1.f / float(p.dim);

    float s[kNSB][VE], dy[kNSB][VE];
    for (int64_t row = row0; row < p.rows; row += rstride) {
        const T* sr = static_cast<const T*>(p.s) + row * p.s_rs;
        const T* dyr = static_cast<const T*>(p.dy) + row * p.dy_rs;
        const T* drr = p.dr ? static_cast<const T*>(p.dr) + row * p.dr_rs : nullptr;
        T* dxr = static_cast<T*>(p.dx) + row * p.dx_rs;
        const float rstd = p.rstd[row];

        // s and dout of segment g into registers; returns this lane's sum of g * s
        auto load_seg = [&](int g) {
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < kNSB; ++k) {
                const int64_t vi = (int64_t(g) * kNSB + k) * 64 + lane;
                if (vi < nvec) {
                    vload<T, VE>(sr + vi * VE, s[k]);
                    vload<T, VE>(dyr + vi * VE, dy[k]);
                    float w1[VE];
                    load_w1<TW, VE>(w, vi, w1);
#pragma unroll
                    for (int e = 0; e < VE; ++e) acc = __builtin_fmaf(dy[k][e] * w1[e], s[k][e], acc);
                }
            }
            return acc;
        };

        float dot = 0.f;
        for (int g = 0; g < nseg; ++g) dot += load_seg(g);
        dot = wave_sum(dot);
        const float c = rstd * rstd * rstd * dot * inv_dim;

        for (int g = nseg - 1; g >= 0; --g) {
            if (g != nseg - 1) (void)load_seg(g);
#pragma unroll
            for (int k = 0; k < kNSB; ++k) {
                const int64_t vi = (int64_t(g) * kNSB + k) * 64 + lane;
                if (vi < nvec) {
                    float w1[VE], o[VE];
                    load_w1<TW, VE>(w, vi, w1);
#pragma unroll
                    for (int e = 0; e < VE; ++e) o[e] = rstd * (dy[k][e] * w1[e]) - c * s[k][e];
                    if (drr) {
                        float dr[VE];
                        vload<T, VE>(drr + vi * VE, dr);
#pragma unroll
                        for (int e = 0; e < VE; ++e) o[e] += dr[e];
                    }
                    vstore<T, VE>(dxr + vi * VE, o);
#pragma unroll
                    for (int e = 0; e < VE; ++e) s_dw[e * nvec + vi] += dy[k][e] * (s[k][e] * rstd);
                }
            }
        }
    }
}

// Each wave of the workgroup (blockDim.x / 64 of them, at most kBwdWaves)
// sums its rows' dweight terms into its own LDS region of dim floats;
// column c = vi * VE + e lives at region[e * nvec + vi], so the 64 lanes of
// one LDS access touch 64 consecutive words (no bank conflicts).  The
// workgroup then writes region 0 + region 1 + ... (in wave order) to its
// row of the workspace, so every sum has a fixed order and dweight is the
// same bits on every run.  kResident: every row fits one register segment
// (bwd_rows_resident), else bwd_rows_general.
template <typename T, typename TW, int VE, bool kResident>
__global__ __launch_bounds__(64 * kBwdWaves) void rmsnorm_bwd_kernel(const NormParams p) {
    extern __shared__ float s_dw[];                     // (waves, dim) column sums of each wave
    const int nw = int(blockDim.x >> 6);
    for (int64_t c = threadIdx.x; c < int64_t(nw) * p.dim; c += blockDim.x) s_dw[c] = 0.f;
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = int(threadIdx.x >> 6);
    const int64_t nvec = p.dim / VE;
    const int64_t row0 = int64_t(blockIdx.x) * nw + wave;
    const int64_t rstride = int64_t(gridDim.x) * nw;
    float* region = s_dw + int64_t(wave) * p.dim;
    if constexpr (kResident) bwd_rows_resident<T, TW, VE>(p, region, lane, nvec, row0, rstride);
    else bwd_rows_general<T, TW, VE>(p, region, lane, nvec, row0, rstride);

    __syncthreads();
    float* part = p.part + int64_t(blockIdx.x) * p.dim;
    for (int64_t c = threadIdx.x; c < p.dim; c += blockDim.x) {
        const int64_t i = (c % VE) * nvec + c / VE;
        float t = s_dw[i];
        for (int w = 1; w < nw; ++w) t += s_dw[int64_t(w) * p.dim + i];
        part[c] = t;
    }
}

// waves per backward workgroup: kBwdWaves while their LDS regions (one row
// of dim floats each) fit 64 KiB, fewer for longer rows
int bwd_waves(int64_t dim) {
    int nw = kBwdWaves;
    while (nw > 1 && int64_t(nw) * dim * int64_t(sizeof(float)) > 65536) nw >>= 1;
    return nw;
}

// dweight[c] = sum over the nparts rows of part, in a fixed order: wave i of
// a workgroup sums rows i, i + kRedWaves, ... of 64 columns, then wave 0
// adds the kRedWaves sums in order
template <typename TW>
__global__ __launch_bounds__(64 * kRedWaves) void rmsnorm_dw_reduce(const float* part, int64_t nparts, int64_t dim,
                                                                      TW* dw) {
    __shared__ float red[kRedWaves][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t col = int64_t(blockIdx.x) * 64 + lane;
    float acc = 0.f;
    if (col < dim) {
#pragma unroll 8
        for (int64_t i = wv; i < nparts; i += kRedWaves) acc += part[i * dim + col];
    }
    red[wv][lane] = acc;
    __syncthreads();
    if (wv == 0 && col < dim) {
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < kRedWaves; ++i) t += red[i][lane];
        io<TW>::store(dw + col, t);
    }
}

template <typename T, typename TW>
hipError_t launch_tw(const NormParams& p, bool vec, bool bwd, int64_t nparts, void* dw, hipStream_t stream) {
    constexpr int VE = 16 / sizeof(T);
    if (!bwd) {
        const dim3 grid(unsigned((p.rows + kFwdWaves - 1) / kFwdWaves));
        const bool pre = p.rows <= kRmsNormPreRows && p.dim <= 64 * kNSF * VE;
        // few rows: one row per workgroup, so the rows' cache lines are
        // fetched by as many compute units
        if (vec && pre) hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, TW, VE, true>), dim3(unsigned(p.rows)), dim3(64), 0, stream, p);
        else if (vec) hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, TW, VE, false>), grid, dim3(64 * kFwdWaves), 0, stream, p);
        else hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, TW, 1, false>), grid, dim3(64 * kFwdWaves), 0, stream, p);
        return hipGetLastError();
    }
    const int nw = bwd_waves(p.dim);
    const size_t lds = size_t(nw) * size_t(p.dim) * sizeof(float);
    if (nparts > 0) {
        const dim3 grid{unsigned(nparts)}, block{unsigned(64 * nw)};
        if (vec && p.dim <= 64 * kNSB * VE) hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, TW, VE, true>), grid, block, lds, stream, p);
        else if (vec) hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, TW, VE, false>), grid, block, lds, stream, p);
        else hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, TW, 1, false>), grid, block, lds, stream, p);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((rmsnorm_dw_reduce<TW>), dim3(unsigned((p.dim + 63) / 64)), dim3(64 * kRedWaves), 0, stream,
                       p.part, nparts, p.dim, static_cast<TW*>(dw));
    return hipGetLastError();
}

template <typename T>
hipError_t launch_t(const NormParams& p, int w_dtype, bool vec, bool bwd, int64_t nparts, void* dw,
                    hipStream_t stream) {
    if (w_dtype == SS_F32) return launch_tw<T, float>(p, vec, bwd, nparts, dw, stream);
    return launch_tw<T, T>(p, vec, bwd, nparts, dw, stream);
}

bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

}  // namespace

int64_t rmsnorm_bwd_parts(int64_t rows) {
    const int64_t want = (rows + kBwdWaves - 1) / kBwdWaves;
    return want < kRmsNormMaxParts ? want : kRmsNormMaxParts;
}

hipError_t rmsnorm_launch(const ss_rmsnorm_args* a, const ss_rmsnorm_bwd_args* g, hipStream_t stream) {
    NormParams p{};
    const int dtype = g ? g->dtype : a->dtype;
    const int w_dtype = g ? g->w_dtype : a->w_dtype;
    const int64_t ve = dtype == SS_F32 ? 4 : 8;
    p.rows = g ? g->rows : a->rows;
    p.dim = g ? g->dim : a->dim;
    bool vec = p.dim % ve == 0;
    auto vok = [&](const void* q, int64_t rs) { return q == nullptr || (aligned16(q) && rs % ve == 0); };
    int64_t nparts = 0;
    if (g) {
        p.s_rs = g->s_row_stride; p.dy_rs = g->dout_row_stride;
        p.dr_rs = g->dresidual_out_row_stride; p.dx_rs = g->dx_row_stride;
        p.s = g->s; p.w = g->weight; p.rstd = const_cast<float*>(g->rstd);
        p.dy = g->dout; p.dr = g->dresidual_out; p.dx = g->dx;
        p.part = static_cast<float*>(g->workspace);
        vec = vec && vok(p.s, p.s_rs) && vok(p.dy, p.dy_rs) && vok(p.dr, p.dr_rs) && vok(p.dx, p.dx_rs);
        nparts = rmsnorm_bwd_parts(p.rows);
    } else {
        p.x_rs = a->x_row_stride; p.r_rs = a->residual_row_stride;
        p.o_rs = a->out_row_stride; p.ro_rs = a->residual_out_row_stride;
        p.x = a->x; p.r = a->residual; p.w = a->weight;
        p.out = a->out; p.rout = a->residual ? a->residual_out : nullptr; p.rstd = a->rstd;
        p.eps = a->eps;
        vec = vec && vok(p.x, p.x_rs) && vok(p.r, p.r_rs) && vok(p.out, p.o_rs) && vok(p.rout, p.ro_rs);
    }
    void* dw = g ? g->dweight : nullptr;
    switch (dtype) {
        case SS_F32: return launch_t<float>(p, w_dtype, vec, g != nullptr, nparts, dw, stream);
        case SS_BF16: return launch_t<bf16_t>(p, w_dtype, vec, g != nullptr, nparts, dw, stream);
        case SS_F16: return launch_t<_Float16>(p, w_dtype, vec, g != nullptr, nparts, dw, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace ss
