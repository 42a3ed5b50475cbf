// Decode-size linear layer on gfx950's matrix cores:
//
//   Y[b, n] = sum_k X[b, k] * W[n, k] (+ bias[n])      (nn.Linear's layout)
//
// for the few rows b of a single-token step (the block's in-, x-, delta- and
// out-projections at batch <= 64).  Such a product streams the weight once
// and does little arithmetic per byte; the library GEMMs choose large tiles
// for it and take several times the weight's streaming time.
//
// A workgroup computes a 16 (n) x 16 (b) tile of Y, or one slice of K of
// it, with NW waves that take every NW-th K step; each K step is one MFMA
// with the W tile (16 n x KS k) as A and the X tile (KS k x 16 b) as B.
// With 16-byte aligned rows and k_in a multiple of 32 a K step covers 32 k
// on gfx950's v_mfma_f32_16x16x32_bf16 (or f16):
//   A: lane l holds W[n0 + (l & 15)][8 (l >> 4) .. + 7] (one 16-byte load)
//   B: lane l holds X[b0 + (l & 15)][the same 8 k]
//   D: lane l holds Y[b0 + (l & 15)][n0 + 4 (l >> 4) + v], v = 0..3
// otherwise 16 k on v_mfma_f32_16x16x16_bf16 (or f16), with lane l holding
// W[n0 + (l & 15)][4 (l >> 4) .. + 3] and the same k of its X row (an
// 8-byte load each).  The
// wave count grows with the steps a workgroup has (4, 8 or 16) so that a
// wave requests all its steps before it uses any.  The partial tiles of the
// waves are summed through LDS.
//
// Split K: a workgroup's time grows with the K it covers (measured on a
// 16 x 16 tile: 3.1 us at K = 48, 5.7 at 768, 9.0 at 1536, whatever the
// wave count), and a decode product can have very few tiles (5 for the
// x-projection of a 1536-wide block).  For such shapes (fewer than
// kLinSplitMaxTiles tiles) and a workspace, the K range of a tile is cut
// into slices, one workgroup each; each puts its fp32 partial tile into a
// slot, and the last of a tile's workgroups to arrive (a per-tile counter)
// sums the slots in slice order, so the result does not depend on which
// one finishes last, and puts the counter back to zero for the next call.
// The exchange costs about three dependent atomic round trips and grows
// with the atomics it issues, so it pays only where the tiles are few
// (x-projection, 5 tiles: 9.0 -> 5.25 us with 4 slices, 5.8 with 16; output
// projection, 48 tiles: 9.06 -> 6.04 us with 4; the 192-tile input
// projection loses with 2), and each slot moves as 64-bit swaps of two
// outputs.  It uses atomics only: an agent-scope fence writes back and
// invalidates the
// whole L2 of its XCD, which made every workgroup's weight reads miss (53 us
// instead of 5.7 for the 768 x 3072 input projection).  The counters have a
// fixed region ahead of the partials, so calls of different shapes can
// share a workspace.
//
// Epilogue: the bias is added in fp32 and the result rounded once; with a
// conv update the rounded product of an output n < conv.dim is the input of
// that channel's causal conv step (state shifted in place, conv output
// written to Y).  Rows n >= N and b >= B read as zero (clamped addresses)
// and are not stored, so every access stays in bounds.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/mamba_ss.h"
#include "ss_device.hpp"
#include "ss_kernels.hpp"

namespace ss {

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 b16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ f32x4 mfma16(s16x4 a, s16x4 b, f32x4 c) {
    if constexpr (__is_same(T, bf16_t)) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h16x4, a), __builtin_bit_cast(h16x4, b), c,
                                                     0, 0, 0);
    }
}

// 16 x 16 x 32 product (gfx950): 8 k per lane
template <typename T>
__device__ __forceinline__ f32x4 mfma32(s16x8 a, s16x8 b, f32x4 c) {
    if constexpr (__is_same(T, bf16_t)) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b16x8, a), __builtin_bit_cast(b16x8, b), c,
                                                       0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h16x8, a), __builtin_bit_cast(h16x8, b), c,
                                                      0, 0, 0);
    }
}

// KV elements of a row (KV = 4: 8 bytes, KV = 8: 16 bytes)
template <int KV>
using rowvec = short __attribute__((ext_vector_type(KV)));

// v rounded to T and back to float (round to nearest even)
template <typename T>
__device__ __forceinline__ float round_io(float v) {
    if constexpr (__is_same(T, bf16_t)) return __uint_as_float(uint32_t(io<bf16_t>::round(v)) << 16);
    else return float(_Float16(v));
}

struct LinExtra {
    int64_t ksplit;                    // workgroups per output tile (1: no split)
    int64_t kslice;                    // K elements per slice
    int* counters;                     // per tile, in the workspace
    float* partials;                   // (tile, slice, 256) fp32, in the workspace
    int32_t has_conv, has_norm;
    ss_conv1d_update_args conv;
    ss_rmsnorm_args norm;
};

// 16-byte vector of T <-> 8 floats (bf16 / fp16 only)
template <typename T>
__device__ __forceinline__ void unpack8(const uint4& v, float (&o)[8]) {
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

template <typename T>
__device__ __forceinline__ uint32_t pack2_io(float lo, float hi) {
    if constexpr (__is_same(T, bf16_t)) {
        return io<bf16_t>::pack2(lo, hi);
    } else {
        return uint32_t(__builtin_bit_cast(uint16_t, _Float16(lo))) |
               (uint32_t(__builtin_bit_cast(uint16_t, _Float16(hi))) << 16);
    }
}

template <typename T>
__device__ __forceinline__ uint4 pack8(const float (&v)[8]) {
    return make_uint4(pack2_io<T>(v[0], v[1]), pack2_io<T>(v[2], v[3]), pack2_io<T>(v[4], v[5]),
                      pack2_io<T>(v[6], v[7]));
}

// Rows b0 .. b0 + 15 of the RMSNorm input (x + residual) normalised into xs
// (rows of ld elements), one wave per row, with the arithmetic of the
// RMSNorm forward kernel for a row of one register segment: lane l owns the
// 8-element vectors l and l + 64 of the row (k_in <= 1024), sums s^2 with
// fmas in element order and then over the wave by xor shuffles, and
// rounds s = x + residual and the output to T the same way, so the rows
// equal that kernel's output bit for bit.  With write_s, s goes to
// residual_out (and 1 / rms to rstd).
template <typename T>
__device__ __forceinline__ void norm_rows(const ss_rmsnorm_args& n, int64_t b0, int64_t batch, int64_t k_in,
                                          uint16_t* xs, int64_t ld, int w, int nw, int lane, bool write_s) {
    const int64_t nvec = k_in / 8;
    for (int rr = w; rr < 16; rr += nw) {
        const int64_t row = b0 + rr;
        if (row >= batch) break;                       // wave-uniform; no barrier inside
        const T* xr = static_cast<const T*>(n.x) + row * n.x_row_stride;
        const T* rr_ = n.residual ? static_cast<const T*>(n.residual) + row * n.residual_row_stride : nullptr;
        float sv[2][8], w1[2][8];
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int64_t vi = int64_t(k) * 64 + lane;
            if (vi < nvec) {
                if (n.w_dtype == SS_F32) {
                    const float4* wp = reinterpret_cast<const float4*>(static_cast<const float*>(n.weight) + vi * 8);
                    const float4 w0 = wp[0], w4 = wp[1];
                    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) w1[k][e] = 1.f + wv[e];
                } else {
                    float wv[8];
                    unpack8<T>(*reinterpret_cast<const uint4*>(static_cast<const T*>(n.weight) + vi * 8), wv);
#pragma unroll
                    for (int e = 0; e < 8; ++e) w1[k][e] = 1.f + wv[e];
                }
                unpack8<T>(*reinterpret_cast<const uint4*>(xr + vi * 8), sv[k]);
                if (rr_) {
                    float rv[8];
                    unpack8<T>(*reinterpret_cast<const uint4*>(rr_ + vi * 8), rv);
#pragma unroll
                    for (int e = 0; e < 8; ++e) sv[k][e] = round_io<T>(sv[k][e] + rv[e]);
                    if (write_s && n.residual_out)
                        *reinterpret_cast<uint4*>(static_cast<T*>(n.residual_out) + row * n.residual_out_row_stride +
                                                  vi * 8) = pack8<T>(sv[k]);
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(sv[k][e], sv[k][e], acc);
            }
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
        const float rstd = rsqrtf(acc / float(k_in) + n.eps);
        if (write_s && n.rstd && lane == 0) n.rstd[row] = rstd;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int64_t vi = int64_t(k) * 64 + lane;
            if (vi < nvec) {
                float o[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = (sv[k][e] * rstd) * w1[k][e];
                *reinterpret_cast<uint4*>(xs + rr * ld + vi * 8) = pack8<T>(o);
            }
        }
    }
}

// kNorm: the input rows are computed in the kernel by the RMSNorm of
// e.norm (x + residual) and read from LDS (extern xs, 16 rows of k_in + 8
// elements: the padding puts the 16 rows of a 16-byte read on different
// banks)
template <typename T, int NW, int KV, bool kNorm>
__global__ __launch_bounds__(64 * NW) void decode_linear_kernel(const ss_decode_linear_args a, const LinExtra e) {
    constexpr int KS = 4 * KV;                        // k per step: 16 or 32
    constexpr int kBatch = KV == 8 ? 8 : 16;          // steps of a wave in flight at once
    __shared__ float part[NW * 256];
    __shared__ int last;
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int i = lane & 15, q = lane >> 4;
    const int64_t tile_n = blockIdx.x / e.ksplit, kidx = blockIdx.x % e.ksplit;
    const int64_t n0 = tile_n * 16, b0 = int64_t(blockIdx.y) * 16;
    const int64_t n = n0 + i, b = b0 + i;
    const bool nv = n < a.n_out, bv = b < a.batch;
    const uint16_t* wrow = static_cast<const uint16_t*>(a.weight) + (nv ? n : 0) * a.w_row_stride + KV * q;
    const int64_t xld = a.k_in + 8;
    const uint16_t* xrow = kNorm ? xs + i * xld + KV * q
                                 : static_cast<const uint16_t*>(a.x) + (bv ? b : 0) * a.x_row_stride + KV * q;
    // this workgroup's K steps: [kb, ke) (slices are whole steps)
    const int64_t kb = kidx * e.kslice / KS;
    const int64_t kend = (kidx + 1) * e.kslice < a.k_in ? (kidx + 1) * e.kslice : a.k_in;
    const int64_t ke = kend / KS;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    // kBatch steps of this wave are requested before any is used; steps past
    // the end read the last step again and are zeroed
    rowvec<KV> av[kBatch], xv[kBatch];
    auto load_w = [&](int64_t kt0) {
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int64_t kt = kt0 + NW * u;
            const int64_t kc = kt < ke ? kt : ke - 1;
            av[u] = *reinterpret_cast<const rowvec<KV>*>(wrow + kc * KS);
        }
    };
    if constexpr (kNorm) {
        // the first batch of weights is requested before the rows are
        // normalised, so the two waits for memory overlap
        if (kb + w < ke) load_w(kb + w);
        norm_rows<T>(e.norm, b0, a.batch, a.k_in, xs, xld, w, NW, lane, blockIdx.x == 0);
        __syncthreads();
    }
    for (int64_t kt0 = kb + w; kt0 < ke; kt0 += NW * kBatch) {
        if (!kNorm || kt0 != kb + w) load_w(kt0);
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int64_t kt = kt0 + NW * u;
            const int64_t kc = kt < ke ? kt : ke - 1;
            xv[u] = *reinterpret_cast<const rowvec<KV>*>(xrow + kc * KS);
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const bool live = kt0 + NW * u < ke;
            const rowvec<KV> z = {};
            const rowvec<KV> av_ = (live && nv) ? av[u] : z, xv_ = (live && bv) ? xv[u] : z;
            if constexpr (KV == 8) {
                acc = mfma32<T>(av_, xv_, acc);
            } else {
                acc = mfma16<T>(av_, xv_, acc);
            }
        }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) part[(w * 64 + lane) * 4 + v] = acc[v];
    __syncthreads();
    // thread t < 256 sums output (lane t / 4, component t % 4) over the waves
    const int t = threadIdx.x;
    float o = 0.f;
    if (t < 256) {
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) o += part[ww * 256 + t];
    }
    if (e.ksplit > 1) {
        // every exchange between the workgroups of a tile is an atomic
        // read-modify-write, performed where the whole device sees it, so no
        // cache write-back or invalidation is needed: the partial goes into
        // its slot by 64-bit atomic swaps (two outputs each), which complete
        // (vmcnt 0) before the counter is advanced; the workgroup that
        // advances it last takes the slots back with atomic swaps (a
        // read-modify-write, which the compiler does not turn into a plain
        // load as it does an OR of 0), in slice order
        const int64_t tile = int64_t(blockIdx.y) * (int64_t(gridDim.x) / e.ksplit) + tile_n;
        unsigned long long* pt = reinterpret_cast<unsigned long long*>(e.partials + tile * e.ksplit * 256);
        if (t < 128) {
            float o0 = 0.f, o1 = 0.f;
#pragma unroll
            for (int ww = 0; ww < NW; ++ww) {
                o0 += part[ww * 256 + 2 * t];
                o1 += part[ww * 256 + 2 * t + 1];
            }
            (void)atomicExch(pt + kidx * 128 + t,
                             (static_cast<unsigned long long>(__float_as_uint(o1)) << 32) | __float_as_uint(o0));
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (t == 0) last = atomicAdd(e.counters + tile, 1) == int(e.ksplit) - 1;
        __syncthreads();
        if (!last) return;
        if (t < 128) {
            // every slot is requested before the first is added (one wait)
            unsigned long long sv[kLinMaxSplit];
#pragma unroll
            for (int k = 0; k < kLinMaxSplit; ++k) sv[k] = k < e.ksplit ? atomicExch(pt + k * 128 + t, 0ull) : 0ull;
            float o0 = 0.f, o1 = 0.f;
#pragma unroll
            for (int k = 0; k < kLinMaxSplit; ++k) {
                o0 += __uint_as_float(uint32_t(sv[k]));
                o1 += __uint_as_float(uint32_t(sv[k] >> 32));
            }
            part[2 * t] = o0;                         // every read of part is behind the barriers above
            part[2 * t + 1] = o1;
        }
        if (t == 0) (void)atomicExch(e.counters + tile, 0);
        __syncthreads();
        if (t < 256) o = part[t];
    }
    if (t >= 256) return;
    const int ol = t >> 2, v = t & 3;
    const int64_t ob = b0 + (ol & 15), on = n0 + 4 * (ol >> 4) + v;
    if (ob >= a.batch || on >= a.n_out) return;
    if (a.bias) {
        o += a.bias_dtype == SS_F32 ? static_cast<const float*>(a.bias)[on]
                                    : io<T>::load(static_cast<const T*>(a.bias) + on);
    }
    if (e.has_conv && on < e.conv.dim) {
        // the causal conv step of channel on, fed the product as it would be
        // stored (rounded to T), in the order of the conv update kernel
        const ss_conv1d_update_args& c = e.conv;
        const int W = int(c.width);
        T* st = static_cast<T*>(c.conv_state) + ob * c.state_batch_stride + on * c.state_dim_stride;
        float sv[4];
        for (int k = 0; k < W - 1; ++k) sv[k] = io<T>::load(st + (k + 1) * c.state_width_stride);
        sv[W - 1] = round_io<T>(o);
        float cacc = c.has_bias ? c.bias[on] : 0.f;
        for (int k = 0; k < W; ++k) {
            cacc = __builtin_fmaf(c.weight[on * c.w_dim_stride + k * c.w_width_stride], sv[k], cacc);
            io<T>::store(st + k * c.state_width_stride, sv[k]);
        }
        if (c.silu) cacc *= sigmoidf_(cacc);
        o = cacc;
    }
    io<T>::store(static_cast<T*>(a.y) + ob * a.y_row_stride + on, o);
}

template <typename T, int KV, bool kNorm>
void launch_kvn(const ss_decode_linear_args* a, const LinExtra& e, hipStream_t stream) {
    const dim3 grid{unsigned((a->n_out + 15) / 16 * e.ksplit), unsigned((a->batch + 15) / 16)};
    const int64_t steps = (e.kslice + 4 * KV - 1) / (4 * KV);   // K steps per workgroup
    const size_t lds = kNorm ? size_t(16 * (a->k_in + 8) * 2) : 0;
    if (steps <= 16) hipLaunchKernelGGL((decode_linear_kernel<T, 4, KV, kNorm>), grid, dim3(256), lds, stream, *a, e);
    else if (steps <= 32) hipLaunchKernelGGL((decode_linear_kernel<T, 8, KV, kNorm>), grid, dim3(512), lds, stream, *a, e);
    else hipLaunchKernelGGL((decode_linear_kernel<T, 16, KV, kNorm>), grid, dim3(1024), lds, stream, *a, e);
}

template <typename T, int KV>
void launch_kv(const ss_decode_linear_args* a, const LinExtra& e, hipStream_t stream) {
    if (e.has_norm) launch_kvn<T, KV, true>(a, e, stream);
    else launch_kvn<T, KV, false>(a, e, stream);
}

template <typename T>
void launch_t(const ss_decode_linear_args* a, const LinExtra& e, hipStream_t stream) {
    // (with the norm the rows come from LDS, 16-byte aligned)
    const bool xok = e.has_norm || (a->x_row_stride % 8 == 0 && (reinterpret_cast<uintptr_t>(a->x) & 15) == 0);
    const bool wide = a->k_in % 32 == 0 && xok && a->w_row_stride % 8 == 0 &&
                      (reinterpret_cast<uintptr_t>(a->weight) & 15) == 0;
    if (wide) launch_kv<T, 8>(a, e, stream);
    else launch_kv<T, 4>(a, e, stream);
}

}  // namespace

DecodeLinearSplit decode_linear_split(int64_t batch, int64_t n_out, int64_t k_in) {
    DecodeLinearSplit sp{1, k_in, 0};
    const int64_t unit = k_in % 32 == 0 ? 32 : 16;               // slices are whole K steps of either kernel
    const int64_t units = k_in / unit;
    const int64_t tiles = ((n_out + 15) / 16) * ((batch + 15) / 16);
    if (tiles <= 0 || units < 4 || tiles >= kLinSplitMaxTiles) return sp;
    const int64_t ks = kLinMaxSplit < units / 2 ? kLinMaxSplit : units / 2;   // at least 2 units per slice
    if (ks < 2) return sp;
    const int64_t per = (units + ks - 1) / ks;
    sp.ksplit = (units + per - 1) / per;
    sp.kslice = per * unit;
    if (sp.ksplit < 2) return DecodeLinearSplit{1, k_in, 0};
    sp.workspace_bytes = kLinCounterBytes + tiles * sp.ksplit * 256 * 4;
    return sp;
}

hipError_t decode_linear_launch(const ss_decode_linear_args* a, hipStream_t stream) {
    LinExtra e{};
    e.ksplit = 1;
    e.kslice = a->k_in;
    const DecodeLinearSplit sp = decode_linear_split(a->batch, a->n_out, a->k_in);
    if (a->workspace && sp.ksplit > 1 && a->workspace_bytes >= sp.workspace_bytes && !a->norm) {
        e.ksplit = sp.ksplit;
        e.kslice = sp.kslice;
        e.counters = static_cast<int*>(a->workspace);
        e.partials = reinterpret_cast<float*>(static_cast<char*>(a->workspace) + kLinCounterBytes);
    }
    if (a->conv) {
        e.has_conv = 1;
        e.conv = *a->conv;
    }
    if (a->norm) {
        e.has_norm = 1;
        e.norm = *a->norm;
    }
    if (a->dtype == SS_BF16) launch_t<bf16_t>(a, e, stream);
    else launch_t<_Float16>(a, e, stream);
    return hipGetLastError();
}

}  // namespace ss
