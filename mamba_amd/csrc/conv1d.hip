// Causal depthwise conv1d (+ SiLU) on gfx950, forward and backward.
//
// The reference runs this step in PyTorch as nn.Conv1d(groups=dim,
// padding=width - 1) cut to the first seqlen outputs, followed by SiLU
// (modules/mamba_simple.py:40-47,100-101):
//
//   pre[b, d, t] = bias[d] + sum_k w[d, k] * x[b, d, t - (width - 1) + k]   (x = 0 before t = 0)
//   out = silu(pre) or pre
//
// Layout: a workgroup of 256 threads covers 256 VW consecutive steps of one
// (batch, channel) row (grid x: rows, grid y: segments); each thread VW
// consecutive steps, one 16-byte vector: VW = 4 for fp32, 8 for 16-bit
// types.  The vectors need only element alignment (this target accesses
// memory in its unaligned mode: 16-byte loads and stores at any element
// offset), so rows at any offset and of any length keep them; the one
// vector that straddles a row's end is read and written element by element.
// The 3-step halo before a thread's steps comes from the previous vector (an
// L1 / L2 hit).
// The op is HBM-bound: one read of x, one write of out (forward); reads of
// x and dout, one write of dx, and per-workgroup sums of dweight / dbias
// (backward).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/mamba_ss.h"
#include "ss_device.hpp"

namespace ss {

namespace {

constexpr int kCT = 256;            // threads per workgroup

struct ConvParams {
    int64_t batch, dim, seqlen;
    int32_t width, has_bias, silu;
    int32_t exact;                               // seqlen a multiple of the vector's steps
    int64_t x_bs, x_ds, o_bs, o_ds, w_ds, w_ks;
    int64_t do_bs, do_ds, dx_bs, dx_ds;
    const void* x; const float* w; const float* bias; void* out;
    const void* dout; void* dx; float* dw; float* dbias;
    float* part;                                 // fixed-order sums: (row, tile, 5) partials; null: atomics
};

template <typename IT>
__device__ __forceinline__ float ld(const IT* p, int64_t i, int64_t n) {
    // element i of a row of n elements; 0 outside [0, n)
    const int64_t c = i < 0 ? 0 : (i >= n ? n - 1 : i);
    const float v = io<IT>::load(p + c);
    return (i >= 0 && i < n) ? v : 0.f;
}

// 16-byte vectors with element alignment only
typedef float f32x4_u __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4_u __attribute__((ext_vector_type(4), aligned(2)));

// VW consecutive elements starting at i (a multiple of VW; 16 bytes: VW = 4
// fp32, 8 16-bit; any element offset); zeros outside [0, n).  kExact: n is
// a multiple of VW, so each vector lies wholly inside or outside the row
// (one load, at a clamped index when outside); otherwise a vector that
// straddles the row's end is read element by element.
template <typename IT, int VW, bool kExact>
__device__ __forceinline__ void ldv(const IT* p, int64_t i, int64_t n, float (&o)[VW]) {
    static_assert(VW * sizeof(IT) == 16, "16-byte vectors");
    const bool in = i >= 0 && i < n;
    if constexpr (!kExact) {
        if (in && i + VW > n) {
#pragma unroll
            for (int k = 0; k < VW; ++k) o[k] = ld<IT>(p, i + k, n);
            return;
        }
    }
    const int64_t c = in ? i : 0;
    if constexpr (sizeof(IT) == 4) {
        const f32x4_u v = *reinterpret_cast<const f32x4_u*>(p + c);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    } else {
        const u32x4_u v = *reinterpret_cast<const u32x4_u*>(p + c);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if constexpr (__is_same(IT, bf16_t)) {
                o[2 * k] = __uint_as_float(w[k] << 16);
                o[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
            } else {
                o[2 * k] = float(__builtin_bit_cast(_Float16, uint16_t(w[k] & 0xffffu)));
                o[2 * k + 1] = float(__builtin_bit_cast(_Float16, uint16_t(w[k] >> 16)));
            }
        }
    }
    if (!in) {
#pragma unroll
        for (int k = 0; k < VW; ++k) o[k] = 0.f;
    }
}

// v into elements i .. i + VW - 1 of a row of n (0 <= i < n): one 16-byte
// store, or (not kExact) element stores of those below n when the vector
// straddles the row's end
template <typename IT, int VW, bool kExact>
__device__ __forceinline__ void stv(IT* p, int64_t i, int64_t n, const float (&v)[VW]) {
    static_assert(VW * sizeof(IT) == 16, "16-byte vectors");
    if (!kExact && i + VW > n) {
#pragma unroll
        for (int k = 0; k < VW; ++k)
            if (i + k < n) io<IT>::store(p + i + k, v[k]);
        return;
    }
    if constexpr (sizeof(IT) == 4) {
        *reinterpret_cast<f32x4_u*>(p + i) = f32x4_u{v[0], v[1], v[2], v[3]};
    } else {
        uint32_t o[VW / 2];
#pragma unroll
        for (int k = 0; k < VW / 2; ++k) {
            if constexpr (__is_same(IT, bf16_t)) {
                o[k] = io<bf16_t>::pack2(v[2 * k], v[2 * k + 1]);
            } else {
                o[k] = uint32_t(__builtin_bit_cast(uint16_t, _Float16(v[2 * k]))) |
                       (uint32_t(__builtin_bit_cast(uint16_t, _Float16(v[2 * k + 1]))) << 16);
            }
        }
        *reinterpret_cast<u32x4_u*>(p + i) = u32x4_u{o[0], o[1], o[2], o[3]};
    }
}

// x[t0 - VW .. t0 + VW * (1 + extra) - 1] into xs
template <typename IT, int VW, bool kExact, int kExtra>
__device__ __forceinline__ void load_window(const IT* row, int64_t t0, int64_t L, float (&xs)[VW * (2 + kExtra)]) {
#pragma unroll
    for (int q = 0; q < 2 + kExtra; ++q) {
        float v[VW];
        ldv<IT, VW, kExact>(row, t0 - VW + VW * q, L, v);
#pragma unroll
        for (int k = 0; k < VW; ++k) xs[VW * q + k] = v[k];
    }
}

template <typename IT, int VW, bool kExact>
__global__ __launch_bounds__(kCT) void conv1d_fwd_kernel(const ConvParams p) {
    constexpr int V = VW;                               // steps per thread
    const int64_t row_id = blockIdx.x;                  // b * dim + d
    const int64_t b = row_id / p.dim, d = row_id % p.dim;
    const int64_t t0 = int64_t(blockIdx.y) * (kCT * V) + threadIdx.x * V;
    if (t0 >= p.seqlen) return;                         // no barrier in this kernel
    const IT* xr = static_cast<const IT*>(p.x) + b * p.x_bs + d * p.x_ds;
    IT* orow = static_cast<IT*>(p.out) + b * p.o_bs + d * p.o_ds;

    float w[4] = {0.f, 0.f, 0.f, 0.f};                  // taps aligned to the right: w[4 - width .. 3]
    for (int k = 0; k < p.width; ++k) w[4 - p.width + k] = p.w[d * p.w_ds + k * p.w_ks];
    const float bias = p.has_bias ? p.bias[d] : 0.f;

    float xs[2 * V];                                    // x[t0 - V .. t0 + V - 1]
    load_window<IT, VW, kExact, 0>(xr, t0, p.seqlen, xs);
    float o[V];
#pragma unroll
    for (int i = 0; i < V; ++i) {
        float acc = bias;
#pragma unroll
        for (int k = 0; k < 4; ++k) acc = __builtin_fmaf(w[k], xs[V + i - 3 + k], acc);
        o[i] = p.silu ? acc * sigmoidf_(acc) : acc;
    }
    stv<IT, VW, kExact>(orow, t0, p.seqlen, o);
}

template <typename IT, int VW, bool kExact>
__global__ __launch_bounds__(kCT) void conv1d_bwd_kernel(const ConvParams p) {
    constexpr int V = VW;                               // steps per thread
    __shared__ float red[kCT / 64][5];
    const int64_t row_id = blockIdx.x;
    const int64_t b = row_id / p.dim, d = row_id % p.dim;
    const int64_t t0 = int64_t(blockIdx.y) * (kCT * V) + threadIdx.x * V;
    const bool live = t0 < p.seqlen;
    const int64_t tl = live ? t0 : 0;                   // dead threads still join the reduction
    const IT* xr = static_cast<const IT*>(p.x) + b * p.x_bs + d * p.x_ds;
    const IT* gr = static_cast<const IT*>(p.dout) + b * p.do_bs + d * p.do_ds;
    IT* dxr = static_cast<IT*>(p.dx) + b * p.dx_bs + d * p.dx_ds;

    float w[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < p.width; ++k) w[4 - p.width + k] = p.w[d * p.w_ds + k * p.w_ks];
    const float bias = p.has_bias ? p.bias[d] : 0.f;

    // x[t0 - V .. t0 + 2 V - 1], dout[t0 .. t0 + 2 V - 1]
    float xs[3 * V];
    load_window<IT, VW, kExact, 1>(xr, tl, p.seqlen, xs);
    float gs[2 * V];
    {
        float v[VW];
        ldv<IT, VW, kExact>(gr, tl, p.seqlen, v);
#pragma unroll
        for (int k = 0; k < VW; ++k) gs[k] = v[k];
        ldv<IT, VW, kExact>(gr, tl + VW, p.seqlen, v);
#pragma unroll
        for (int k = 0; k < VW; ++k) gs[VW + k] = v[k];
    }
    // dpre at t0 .. t0 + 2 V - 1 (zero beyond seqlen: gs is zero there)
    float dp[2 * V];
#pragma unroll
    for (int i = 0; i < 2 * V; ++i) {
        float pre = bias;
#pragma unroll
        for (int k = 0; k < 4; ++k) pre = __builtin_fmaf(w[k], xs[V + i - 3 + k], pre);
        float g = gs[i];
        if (p.silu) {
            const float s = sigmoidf_(pre);
            g *= s * (1.f + pre * (1.f - s));
        }
        dp[i] = g;
    }
    // dx[t] = sum_k w[k] * dpre[t + 3 - k] (taps right-aligned)
    float dxo[V];
#pragma unroll
    for (int i = 0; i < V; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) acc = __builtin_fmaf(w[k], dp[i + 3 - k], acc);
        dxo[i] = acc;
    }
    if (live) stv<IT, VW, kExact>(dxr, t0, p.seqlen, dxo);
    // dw[k] += sum_t dpre[t] * x[t - 3 + k], dbias += sum_t dpre[t], over this thread's V steps
    float part[5];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < V; ++i) acc = __builtin_fmaf(dp[i], xs[V + i - 3 + k], acc);
        part[k] = live ? acc : 0.f;
    }
    {
        float sb = 0.f;
#pragma unroll
        for (int i = 0; i < V; ++i) sb += dp[i];
        part[4] = live ? sb : 0.f;
    }
#pragma unroll
    for (int k = 0; k < 5; ++k) {
        float v = part[k];
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
        part[k] = v;
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < 5; ++k) red[wv][k] = part[k];
    }
    __syncthreads();
    if (threadIdx.x < 5) {
        const int k = threadIdx.x;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < kCT / 64; ++i) s += red[i][k];
        if (p.part) {                                   // summed later in a fixed order
            p.part[(row_id * int64_t(gridDim.y) + blockIdx.y) * 5 + k] = s;
            return;
        }
        if (k < 4) {
            const int tap = k - (4 - p.width);          // right-aligned slot k is tap k - (4 - width)
            if (tap >= 0) atomicAdd(p.dw + d * p.width + tap, s);
        } else if (p.dbias) {
            atomicAdd(p.dbias + d, s);
        }
    }
}

// dweight / dbias += the backward's partials, one thread per (channel, slot
// k): slots 0..3 the right-aligned taps, 4 the bias; summed over batch rows,
// then sequence tiles, in that order
__global__ __launch_bounds__(256) void conv1d_bwd_reduce(const float* __restrict__ part, int64_t batch, int64_t dim,
                                                         int64_t ntiles, int width, float* __restrict__ dw,
                                                         float* __restrict__ dbias) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= dim * 5) return;
    const int64_t d = i / 5;
    const int k = int(i % 5);
    float s = 0.f;
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t t = 0; t < ntiles; ++t) s += part[((b * dim + d) * ntiles + t) * 5 + k];
    if (k < 4) {
        const int tap = k - (4 - width);
        if (tap >= 0) dw[d * width + tap] += s;
    } else if (dbias) {
        dbias[d] += s;
    }
}

template <typename IT, int VW, bool kExact>
void launch_vw(const ConvParams& p, bool bwd, hipStream_t stream) {
    constexpr int V = VW;
    const dim3 grid(unsigned(p.batch * p.dim), unsigned((p.seqlen + kCT * V - 1) / (kCT * V)));
    if (bwd) {
        hipLaunchKernelGGL((conv1d_bwd_kernel<IT, VW, kExact>), grid, dim3(kCT), 0, stream, p);
        if (p.part)
            hipLaunchKernelGGL(conv1d_bwd_reduce, dim3(unsigned((p.dim * 5 + 255) / 256)), dim3(256), 0, stream,
                               p.part, p.batch, p.dim, int64_t(grid.y), int(p.width), p.dw, p.dbias);
    } else {
        hipLaunchKernelGGL((conv1d_fwd_kernel<IT, VW, kExact>), grid, dim3(kCT), 0, stream, p);
    }
}

template <typename IT>
hipError_t launch_t(const ConvParams& p, bool bwd, hipStream_t stream) {
    // 16-byte vectors; rows of whole vectors take the branch-free loads
    if (p.exact) launch_vw<IT, 16 / sizeof(IT), true>(p, bwd, stream);
    else launch_vw<IT, 16 / sizeof(IT), false>(p, bwd, stream);
    return hipGetLastError();
}

hipError_t launch_conv(const ConvParams& p, int itype, bool bwd, hipStream_t stream) {
    switch (itype) {
        case SS_F32: return launch_t<float>(p, bwd, stream);
        case SS_BF16: return launch_t<bf16_t>(p, bwd, stream);
        case SS_F16: return launch_t<_Float16>(p, bwd, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

int64_t conv1d_bwd_workspace_bytes(int64_t batch, int64_t dim, int64_t seqlen) {
    // the most sequence tiles a launch can have (4 steps per thread)
    const int64_t ntiles = (seqlen + kCT * 4 - 1) / (kCT * 4);
    return batch * dim * ntiles * 5 * int64_t(sizeof(float));
}

hipError_t conv1d_launch(const ss_conv1d_args* a, const ss_conv1d_bwd_args* g, hipStream_t stream) {
    ConvParams p{};
    p.batch = a->batch; p.dim = a->dim; p.seqlen = a->seqlen; p.width = int32_t(a->width);
    p.has_bias = a->has_bias; p.silu = a->silu;
    p.x_bs = a->x_batch_stride; p.x_ds = a->x_dim_stride;
    p.o_bs = a->out_batch_stride; p.o_ds = a->out_dim_stride;
    p.w_ds = a->w_dim_stride; p.w_ks = a->w_width_stride;
    p.x = a->x; p.w = a->weight; p.bias = a->has_bias ? a->bias : nullptr; p.out = a->out;
    if (g) {
        p.do_bs = g->dout_batch_stride; p.do_ds = g->dout_dim_stride;
        p.dx_bs = g->dx_batch_stride; p.dx_ds = g->dx_dim_stride;
        p.dout = g->dout; p.dx = g->dx; p.dw = g->dweight; p.dbias = a->has_bias ? g->dbias : nullptr;
        p.part = g->workspace;
    }
    p.exact = p.seqlen % int64_t(a->itype == SS_F32 ? 4 : 8) == 0;
    return launch_conv(p, a->itype, g != nullptr, stream);
}

}  // namespace ss
