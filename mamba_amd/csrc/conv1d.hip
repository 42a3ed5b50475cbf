// Causal depthwise conv1d (+ SiLU) on gfx950, forward and backward.
//
// The reference runs this step in PyTorch as nn.Conv1d(groups=dim,
// padding=width - 1) cut to the first seqlen outputs, followed by SiLU
// (modules/mamba_simple.py:40-47,100-101):
//
//   pre[b, d, t] = bias[d] + sum_k w[d, k] * x[b, d, t - (width - 1) + k]   (x = 0 before t = 0)
//   out = silu(pre) or pre
//
// Layout: a workgroup of 256 threads covers 1024 consecutive steps of one
// (batch, channel) row (grid x: rows, grid y: 1024-step segments); each
// thread 4 consecutive steps.  Rows are read with
// 4-element vector loads when they are 4-element aligned (seqlen and the
// strides multiples of 4), element by element otherwise.  The 3-step halo
// before a thread's steps comes from the previous vector (an L1 / L2 hit).
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
constexpr int kCV = 4;              // steps per thread
constexpr int kCSeg = kCT * kCV;    // steps per workgroup

struct ConvParams {
    int64_t batch, dim, seqlen;
    int32_t width, has_bias, silu, vec;
    int64_t x_bs, x_ds, o_bs, o_ds, w_ds, w_ks;
    int64_t do_bs, do_ds, dx_bs, dx_ds;
    const void* x; const float* w; const float* bias; void* out;
    const void* dout; void* dx; float* dw; float* dbias;
};

template <typename IT>
__device__ __forceinline__ float ld(const IT* p, int64_t i, int64_t n) {
    // element i of a row of n elements; 0 outside [0, n)
    const int64_t c = i < 0 ? 0 : (i >= n ? n - 1 : i);
    const float v = io<IT>::load(p + c);
    return (i >= 0 && i < n) ? v : 0.f;
}

// 4 consecutive elements starting at i (a multiple of 4, 4-element aligned
// row); zeros outside [0, n) (n is a multiple of 4 on this path)
template <typename IT>
__device__ __forceinline__ void ld4(const IT* p, int64_t i, int64_t n, float (&o)[4]) {
    const bool in = i >= 0 && i < n;
    const int64_t c = in ? i : 0;
    if constexpr (sizeof(IT) == 4) {
        const float4 v = *reinterpret_cast<const float4*>(p + c);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    } else {
        const uint2 v = *reinterpret_cast<const uint2*>(p + c);
        const uint32_t w[2] = {v.x, v.y};
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            if constexpr (__is_same(IT, bf16_t)) {
                o[2 * k] = __uint_as_float(w[k] << 16);
                o[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
            } else {
                o[2 * k] = float(__builtin_bit_cast(_Float16, uint16_t(w[k] & 0xffffu)));
                o[2 * k + 1] = float(__builtin_bit_cast(_Float16, uint16_t(w[k] >> 16)));
            }
        }
    }
    if (!in) { o[0] = 0.f; o[1] = 0.f; o[2] = 0.f; o[3] = 0.f; }
}

template <typename IT>
__device__ __forceinline__ void st4(IT* p, float (&v)[4]) {
    if constexpr (sizeof(IT) == 4) {
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    } else if constexpr (__is_same(IT, bf16_t)) {
        *reinterpret_cast<uint2*>(p) = make_uint2(io<bf16_t>::pack2(v[0], v[1]), io<bf16_t>::pack2(v[2], v[3]));
    } else {
        uint2 o;
        o.x = uint32_t(__builtin_bit_cast(uint16_t, _Float16(v[0]))) | (uint32_t(__builtin_bit_cast(uint16_t, _Float16(v[1]))) << 16);
        o.y = uint32_t(__builtin_bit_cast(uint16_t, _Float16(v[2]))) | (uint32_t(__builtin_bit_cast(uint16_t, _Float16(v[3]))) << 16);
        *reinterpret_cast<uint2*>(p) = o;
    }
}

// x[t0 - 4 .. t0 + 4 * extra + 3] into xs[0 .. 4 + 4 * extra + 3]
template <typename IT, bool kVec, int kExtra>
__device__ __forceinline__ void load_window(const IT* row, int64_t t0, int64_t L, float (&xs)[8 + 4 * kExtra]) {
    if constexpr (kVec) {
#pragma unroll
        for (int q = 0; q < 2 + kExtra; ++q) {
            float v[4];
            ld4<IT>(row, t0 - 4 + 4 * q, L, v);
#pragma unroll
            for (int k = 0; k < 4; ++k) xs[4 * q + k] = v[k];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8 + 4 * kExtra; ++i) xs[i] = ld<IT>(row, t0 - 4 + i, L);
    }
}

template <typename IT, bool kVec>
__global__ __launch_bounds__(kCT) void conv1d_fwd_kernel(const ConvParams p) {
    const int64_t row_id = blockIdx.x;                  // b * dim + d
    const int64_t b = row_id / p.dim, d = row_id % p.dim;
    const int64_t t0 = int64_t(blockIdx.y) * kCSeg + threadIdx.x * kCV;
    if (t0 >= p.seqlen) return;                         // no barrier in this kernel
    const IT* xr = static_cast<const IT*>(p.x) + b * p.x_bs + d * p.x_ds;
    IT* orow = static_cast<IT*>(p.out) + b * p.o_bs + d * p.o_ds;

    float w[4] = {0.f, 0.f, 0.f, 0.f};                  // taps aligned to the right: w[4 - width .. 3]
    for (int k = 0; k < p.width; ++k) w[4 - p.width + k] = p.w[d * p.w_ds + k * p.w_ks];
    const float bias = p.has_bias ? p.bias[d] : 0.f;

    float xs[8];
    load_window<IT, kVec, 0>(xr, t0, p.seqlen, xs);
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float acc = bias;
#pragma unroll
        for (int k = 0; k < 4; ++k) acc = __builtin_fmaf(w[k], xs[i + 1 + k], acc);
        o[i] = p.silu ? acc * sigmoidf_(acc) : acc;
    }
    if constexpr (kVec) {
        st4<IT>(orow + t0, o);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (t0 + i < p.seqlen) io<IT>::store(orow + t0 + i, o[i]);
    }
}

template <typename IT, bool kVec>
__global__ __launch_bounds__(kCT) void conv1d_bwd_kernel(const ConvParams p) {
    __shared__ float red[kCT / 64][5];
    const int64_t row_id = blockIdx.x;
    const int64_t b = row_id / p.dim, d = row_id % p.dim;
    const int64_t t0 = int64_t(blockIdx.y) * kCSeg + threadIdx.x * kCV;
    const bool live = t0 < p.seqlen;
    const int64_t tl = live ? t0 : 0;                   // dead threads still join the reduction
    const IT* xr = static_cast<const IT*>(p.x) + b * p.x_bs + d * p.x_ds;
    const IT* gr = static_cast<const IT*>(p.dout) + b * p.do_bs + d * p.do_ds;
    IT* dxr = static_cast<IT*>(p.dx) + b * p.dx_bs + d * p.dx_ds;

    float w[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < p.width; ++k) w[4 - p.width + k] = p.w[d * p.w_ds + k * p.w_ks];
    const float bias = p.has_bias ? p.bias[d] : 0.f;

    // x[t0 - 4 .. t0 + 7], dout[t0 .. t0 + 7]
    float xs[12];
    load_window<IT, kVec, 1>(xr, tl, p.seqlen, xs);
    float gs[8];
    if constexpr (kVec) {
        float v[4];
        ld4<IT>(gr, tl, p.seqlen, v);
#pragma unroll
        for (int k = 0; k < 4; ++k) gs[k] = v[k];
        ld4<IT>(gr, tl + 4, p.seqlen, v);
#pragma unroll
        for (int k = 0; k < 4; ++k) gs[4 + k] = v[k];
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) gs[i] = ld<IT>(gr, tl + i, p.seqlen);
    }
    // dpre at t0 .. t0 + 7 (zero beyond seqlen: gs is zero there)
    float dp[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float pre = bias;
#pragma unroll
        for (int k = 0; k < 4; ++k) pre = __builtin_fmaf(w[k], xs[i + 1 + k], pre);
        float g = gs[i];
        if (p.silu) {
            const float s = sigmoidf_(pre);
            g *= s * (1.f + pre * (1.f - s));
        }
        dp[i] = g;
    }
    // dx[t] = sum_k w[k] * dpre[t + 3 - k] (taps right-aligned)
    float dxo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) acc = __builtin_fmaf(w[k], dp[i + 3 - k], acc);
        dxo[i] = acc;
    }
    if (live) {
        if constexpr (kVec) {
            st4<IT>(dxr + t0, dxo);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (t0 + i < p.seqlen) io<IT>::store(dxr + t0 + i, dxo[i]);
        }
    }
    // dw[k] += sum_t dpre[t] * x[t - 3 + k], dbias += sum_t dpre[t], over this thread's 4 steps
    float part[5];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = __builtin_fmaf(dp[i], xs[i + 1 + k], acc);
        part[k] = live ? acc : 0.f;
    }
    part[4] = live ? dp[0] + dp[1] + dp[2] + dp[3] : 0.f;
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
        if (k < 4) {
            const int tap = k - (4 - p.width);          // right-aligned slot k is tap k - (4 - width)
            if (tap >= 0) atomicAdd(p.dw + d * p.width + tap, s);
        } else if (p.dbias) {
            atomicAdd(p.dbias + d, s);
        }
    }
}

template <typename IT>
hipError_t launch_t(const ConvParams& p, bool bwd, hipStream_t stream) {
    const dim3 grid(unsigned(p.batch * p.dim), unsigned((p.seqlen + kCSeg - 1) / kCSeg));
    if (bwd) {
        if (p.vec) hipLaunchKernelGGL((conv1d_bwd_kernel<IT, true>), grid, dim3(kCT), 0, stream, p);
        else hipLaunchKernelGGL((conv1d_bwd_kernel<IT, false>), grid, dim3(kCT), 0, stream, p);
    } else {
        if (p.vec) hipLaunchKernelGGL((conv1d_fwd_kernel<IT, true>), grid, dim3(kCT), 0, stream, p);
        else hipLaunchKernelGGL((conv1d_fwd_kernel<IT, false>), grid, dim3(kCT), 0, stream, p);
    }
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

hipError_t conv1d_launch(const ss_conv1d_args* a, const ss_conv1d_bwd_args* g, hipStream_t stream) {
    ConvParams p{};
    p.batch = a->batch; p.dim = a->dim; p.seqlen = a->seqlen; p.width = int32_t(a->width);
    p.has_bias = a->has_bias; p.silu = a->silu;
    p.x_bs = a->x_batch_stride; p.x_ds = a->x_dim_stride;
    p.o_bs = a->out_batch_stride; p.o_ds = a->out_dim_stride;
    p.w_ds = a->w_dim_stride; p.w_ks = a->w_width_stride;
    p.x = a->x; p.w = a->weight; p.bias = a->has_bias ? a->bias : nullptr; p.out = a->out;
    const size_t es = a->itype == SS_F32 ? 4 : 2;
    auto al = [&](const void* q) { return (reinterpret_cast<uintptr_t>(q) % (4 * es)) == 0; };
    bool vec = p.seqlen % 4 == 0 && al(a->x) && p.x_bs % 4 == 0 && p.x_ds % 4 == 0;
    if (g) {
        p.do_bs = g->dout_batch_stride; p.do_ds = g->dout_dim_stride;
        p.dx_bs = g->dx_batch_stride; p.dx_ds = g->dx_dim_stride;
        p.dout = g->dout; p.dx = g->dx; p.dw = g->dweight; p.dbias = a->has_bias ? g->dbias : nullptr;
        vec = vec && al(g->dout) && al(g->dx) && p.do_bs % 4 == 0 && p.do_ds % 4 == 0 &&
              p.dx_bs % 4 == 0 && p.dx_ds % 4 == 0;
    } else {
        vec = vec && al(a->out) && p.o_bs % 4 == 0 && p.o_ds % 4 == 0;
    }
    p.vec = vec;
    return launch_conv(p, a->itype, g != nullptr, stream);
}

}  // namespace ss
