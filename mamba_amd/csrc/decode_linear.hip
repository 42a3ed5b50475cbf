// Decode-size linear layer on gfx950's matrix cores:
//
//   Y[b, n] = sum_k X[b, k] * W[n, k] (+ bias[n])      (nn.Linear's layout)
//
// for the few rows b of a single-token step (the block's in-, x-, delta- and
// out-projections at batch <= 64).  Such a product streams the weight once
// and does little arithmetic per byte; the library GEMMs choose large tiles
// for it and take several times the weight's streaming time.
//
// A workgroup computes a 16 (n) x 16 (b) tile of Y.  Its 4 waves take every
// 4th 16-wide step of K; each step is one v_mfma_f32_16x16x16_bf16 (or f16)
// with the W tile (16 n x 16 k) as A and the X tile (16 k x 16 b) as B:
//   A: lane l holds W[n0 + (l & 15)][k + 4 (l >> 4) .. + 3]
//   B: lane l holds X[b0 + (l & 15)][k + 4 (l >> 4) .. + 3]
//   D: lane l holds Y[b0 + (l & 15)][n0 + 4 (l >> 4) + v], v = 0..3
// The 4 partial tiles are summed through LDS; the bias is added in fp32 and
// the result rounded once.  Rows n >= N and b >= B read as zero (clamped
// addresses) and are not stored, so every access stays in bounds.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/mamba_ss.h"
#include "ss_device.hpp"
#include "ss_kernels.hpp"

namespace ss {

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kLinWaves = 4;
constexpr int kLinBatch = 16;          // K steps per wave in flight at once

template <typename T>
__device__ __forceinline__ f32x4 mfma16(s16x4 a, s16x4 b, f32x4 c) {
    if constexpr (__is_same(T, bf16_t)) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h16x4, a), __builtin_bit_cast(h16x4, b), c,
                                                     0, 0, 0);
    }
}

template <typename T>
__global__ __launch_bounds__(64 * kLinWaves) void decode_linear_kernel(const ss_decode_linear_args a) {
    __shared__ f32x4 part[kLinWaves][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int i = lane & 15, q = lane >> 4;
    const int64_t n0 = int64_t(blockIdx.x) * 16, b0 = int64_t(blockIdx.y) * 16;
    const int64_t n = n0 + i, b = b0 + i;
    const bool nv = n < a.n_out, bv = b < a.batch;
    // 4 consecutive elements (8 bytes) of this lane's W row and X row per K step
    const uint16_t* wrow = static_cast<const uint16_t*>(a.weight) + (nv ? n : 0) * a.w_row_stride + 4 * q;
    const uint16_t* xrow = static_cast<const uint16_t*>(a.x) + (bv ? b : 0) * a.x_row_stride + 4 * q;
    const int64_t ksteps = a.k_in / 16;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    // kLinBatch steps of this wave are requested before any is used, so a
    // wave waits for memory once per batch (once in all for k_in <= 1024);
    // steps past the end read the last step again and are zeroed
    for (int64_t kt0 = w; kt0 < ksteps; kt0 += kLinWaves * kLinBatch) {
        s16x4 av[kLinBatch], xv[kLinBatch];
#pragma unroll
        for (int u = 0; u < kLinBatch; ++u) {
            const int64_t kt = kt0 + kLinWaves * u;
            const int64_t kc = kt < ksteps ? kt : ksteps - 1;
            av[u] = *reinterpret_cast<const s16x4*>(wrow + kc * 16);
            xv[u] = *reinterpret_cast<const s16x4*>(xrow + kc * 16);
        }
#pragma unroll
        for (int u = 0; u < kLinBatch; ++u) {
            const bool live = kt0 + kLinWaves * u < ksteps;
            const s16x4 z = {0, 0, 0, 0};
            acc = mfma16<T>((live && nv) ? av[u] : z, (live && bv) ? xv[u] : z, acc);
        }
    }
    part[w][lane] = acc;
    __syncthreads();
    if (w != 0) return;
    f32x4 s = part[0][lane];
#pragma unroll
    for (int ww = 1; ww < kLinWaves; ++ww) s += part[ww][lane];
    if (!bv) return;
    T* yrow = static_cast<T*>(a.y) + b * a.y_row_stride;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int64_t nn = n0 + 4 * q + v;
        if (nn < a.n_out) {
            float o = s[v];
            if (a.bias) {
                o += a.bias_dtype == SS_F32 ? static_cast<const float*>(a.bias)[nn]
                                            : io<T>::load(static_cast<const T*>(a.bias) + nn);
            }
            io<T>::store(yrow + nn, o);
        }
    }
}

template <typename T>
void launch_t(const ss_decode_linear_args* a, hipStream_t stream) {
    const dim3 grid{unsigned((a->n_out + 15) / 16), unsigned((a->batch + 15) / 16)};
    hipLaunchKernelGGL((decode_linear_kernel<T>), grid, dim3(64 * kLinWaves), 0, stream, *a);
}

}  // namespace

hipError_t decode_linear_launch(const ss_decode_linear_args* a, hipStream_t stream) {
    if (a->dtype == SS_BF16) launch_t<bf16_t>(a, stream);
    else launch_t<_Float16>(a, stream);
    return hipGetLastError();
}

}  // namespace ss
