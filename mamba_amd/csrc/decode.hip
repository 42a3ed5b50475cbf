// Single-token decode on gfx950: the selective-scan state update and the
// causal conv1d state update.
//
// The reference has no decode path (CausalLM.generate is a stub,
// models/causal_lm.py:61-62); these kernels advance the recurrences that the
// scan (forward_kernel.cu:216-293) and the block's conv
// (modules/mamba_simple.py:40-47,100-101) compute over a whole sequence by
// one step, from a state kept between steps:
//
//   conv:  state <- (state[1:], x);  out = act(bias + sum_k w[k] * state[k])
//   scan:  delta' = softplus(delta + bias);  h[n] <- exp(delta' A[n]) h[n] + delta' x B[n]
//          y = sum_n C[n] h[n] + D x;  out = y * silu(z)
//
// One thread per (batch, channel): a decode step touches B * D * (N + a few)
// values, so the launch is small and latency-bound; the state row of a
// channel (N fp32) is read and written with 16-byte accesses when it is
// contiguous and aligned.  The exp is computed as exp2(delta' * A * log2 e)
// and the softplus with the threshold at 20, as in the scan kernels.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/mamba_ss.h"
#include "ss_device.hpp"
#include "ss_kernels.hpp"

namespace ss {

namespace {

constexpr int kDT = 256;              // threads per workgroup

template <typename IT>
__global__ __launch_bounds__(kDT) void state_update_kernel(const ss_state_update_args a, bool vec) {
    const int64_t i = int64_t(blockIdx.x) * kDT + threadIdx.x;
    if (i >= a.batch * a.dim) return;                   // no barrier in this kernel
    const int64_t b = i / a.dim, d = i % a.dim;
    const int64_t g = d / (a.dim / a.n_groups);
    const IT* xs = static_cast<const IT*>(a.x);
    const IT* dts = static_cast<const IT*>(a.delta);
    const float x = io<IT>::load(xs + b * a.x_batch_stride + d * a.x_dim_stride);
    float dt = io<IT>::load(dts + b * a.delta_batch_stride + d * a.delta_dim_stride);
    if (a.has_delta_bias) dt += a.delta_bias[d];
    if (a.delta_softplus) dt = softplus20(dt);
    const float dtx = dt * x;
    const IT* Bp = static_cast<const IT*>(a.B) + b * a.B_batch_stride + g * a.B_group_stride;
    const IT* Cp = static_cast<const IT*>(a.C) + b * a.C_batch_stride + g * a.C_group_stride;
    const float* Ap = a.A + d * a.A_dim_stride;
    float* h = a.state + b * a.state_batch_stride + d * a.state_dim_stride;

    float y = 0.f;
    if (vec) {                                          // state, A rows contiguous and 16-byte aligned
        for (int64_t n = 0; n < a.dstate; n += 4) {
            float4 hv = *reinterpret_cast<const float4*>(h + n);
            const float4 av = *reinterpret_cast<const float4*>(Ap + n);
            float hn[4] = {hv.x, hv.y, hv.z, hv.w};
            const float an[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float dA = __builtin_amdgcn_exp2f(dt * an[k] * kLog2e);
                hn[k] = __builtin_fmaf(dA, hn[k], dtx * io<IT>::load(Bp + (n + k) * a.B_dstate_stride));
                y = __builtin_fmaf(io<IT>::load(Cp + (n + k) * a.C_dstate_stride), hn[k], y);
            }
            hv = make_float4(hn[0], hn[1], hn[2], hn[3]);
            *reinterpret_cast<float4*>(h + n) = hv;
        }
    } else {
        for (int64_t n = 0; n < a.dstate; ++n) {
            float* hp = h + n * a.state_dstate_stride;
            const float dA = __builtin_amdgcn_exp2f(dt * Ap[n * a.A_dstate_stride] * kLog2e);
            const float hn = __builtin_fmaf(dA, *hp, dtx * io<IT>::load(Bp + n * a.B_dstate_stride));
            *hp = hn;
            y = __builtin_fmaf(io<IT>::load(Cp + n * a.C_dstate_stride), hn, y);
        }
    }
    if (a.has_D) y = __builtin_fmaf(a.D[d], x, y);
    if (a.has_z) {
        const float z = io<IT>::load(static_cast<const IT*>(a.z) + b * a.z_batch_stride + d * a.z_dim_stride);
        y *= z * sigmoidf_(z);
    }
    io<IT>::store(static_cast<IT*>(a.out) + b * a.out_batch_stride + d * a.out_dim_stride, y);
}

template <typename IT>
__global__ __launch_bounds__(kDT) void conv_update_kernel(const ss_conv1d_update_args a) {
    const int64_t i = int64_t(blockIdx.x) * kDT + threadIdx.x;
    if (i >= a.batch * a.dim) return;                   // no barrier in this kernel
    const int64_t b = i / a.dim, d = i % a.dim;
    const int W = int(a.width);
    IT* st = static_cast<IT*>(a.conv_state) + b * a.state_batch_stride + d * a.state_dim_stride;
    float s[4];
    for (int k = 0; k < W - 1; ++k) s[k] = io<IT>::load(st + (k + 1) * a.state_width_stride);
    s[W - 1] = io<IT>::load(static_cast<const IT*>(a.x) + b * a.x_batch_stride + d * a.x_dim_stride);
    float acc = a.has_bias ? a.bias[d] : 0.f;
    for (int k = 0; k < W; ++k) {
        acc = __builtin_fmaf(a.weight[d * a.w_dim_stride + k * a.w_width_stride], s[k], acc);
        io<IT>::store(st + k * a.state_width_stride, s[k]);
    }
    if (a.silu) acc *= sigmoidf_(acc);
    io<IT>::store(static_cast<IT*>(a.out) + b * a.out_batch_stride + d * a.out_dim_stride, acc);
}

bool al16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

}  // namespace

hipError_t state_update_launch(const ss_state_update_args* a, hipStream_t stream) {
    const bool vec = a->dstate % 4 == 0 && a->state_dstate_stride == 1 && a->A_dstate_stride == 1 &&
                     al16(a->state) && al16(a->A) && a->state_batch_stride % 4 == 0 &&
                     a->state_dim_stride % 4 == 0 && a->A_dim_stride % 4 == 0;
    const dim3 grid{unsigned((a->batch * a->dim + kDT - 1) / kDT)};
    switch (a->itype) {
        case SS_F32: hipLaunchKernelGGL((state_update_kernel<float>), grid, dim3(kDT), 0, stream, *a, vec); break;
        case SS_BF16: hipLaunchKernelGGL((state_update_kernel<bf16_t>), grid, dim3(kDT), 0, stream, *a, vec); break;
        case SS_F16: hipLaunchKernelGGL((state_update_kernel<_Float16>), grid, dim3(kDT), 0, stream, *a, vec); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t conv_update_launch(const ss_conv1d_update_args* a, hipStream_t stream) {
    const dim3 grid{unsigned((a->batch * a->dim + kDT - 1) / kDT)};
    switch (a->itype) {
        case SS_F32: hipLaunchKernelGGL((conv_update_kernel<float>), grid, dim3(kDT), 0, stream, *a); break;
        case SS_BF16: hipLaunchKernelGGL((conv_update_kernel<bf16_t>), grid, dim3(kDT), 0, stream, *a); break;
        case SS_F16: hipLaunchKernelGGL((conv_update_kernel<_Float16>), grid, dim3(kDT), 0, stream, *a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace ss
