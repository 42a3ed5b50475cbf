// Device-side helpers shared by the forward and backward selective-scan
// kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>
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
constexpr int kChunk = 16;        // steps per checkpoint of the state h
constexpr int kMaxSPL = 16;       // state groups: dstate <= 16 * kMaxSPL = 256
constexpr int kXcds = 8;          // accelerator complex dies of an MI355X
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
    // round to nearest even (NaN stays NaN): gfx950's v_cvt_pk_bf16_f32
    static __device__ __forceinline__ uint16_t round(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }
    // two values rounded and packed, lo in bits 0-15, by one v_cvt_pk_bf16_f32
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
        typedef float f2 __attribute__((ext_vector_type(2)));
        typedef __bf16 b2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{lo, hi}, b2));
    }
    static __device__ __forceinline__ void store(bf16_t* p, float v) { p->bits = round(v); }
};
template <> struct io<_Float16> {
    static __device__ __forceinline__ float load(const _Float16* p) { return float(*p); }
    static __device__ __forceinline__ void store(_Float16* p, float v) { *p = _Float16(v); }
};

// Element p[t] as float (t known to be in range).
template <typename T>
__device__ __forceinline__ float load_at(const T* __restrict__ p, int64_t t) { return io<T>::load(p + t); }

// Element p[t] as float, or 0 when t >= L.  The address is clamped to the
// last element so the load is unconditional (no branch, no divergence).
template <typename T>
__device__ __forceinline__ float load_or0(const T* __restrict__ p, int64_t t, int64_t L) {
    const float v = io<T>::load(p + (t < L ? t : L - 1));
    return t < L ? v : 0.f;
}

// Loads row[t0 .. t0+15] as float; steps >= L read as 0.  `vec` says
// row + t0 is 16-byte aligned; full tiles then use 16-byte loads.  The
// branch depends only on uniform values, so no lane waits on another.
template <typename T>
__device__ __forceinline__ void load_tile16(const T* __restrict__ row, int64_t t0, int64_t L, bool vec,
                                            float (&o)[16]) {
    const T* p = row + t0;
    if (vec && t0 + 16 <= L) {
        if constexpr (sizeof(T) == 4) {
            const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = q[i];
                o[4 * i] = v.x; o[4 * i + 1] = v.y; o[4 * i + 2] = v.z; o[4 * i + 3] = v.w;
            }
        } else {
            const uint4* q = reinterpret_cast<const uint4*>(p);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint4 v = q[i];
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if constexpr (__is_same(T, bf16_t)) {
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
        for (int i = 0; i < 16; ++i) o[i] = load_or0(row, t0 + i, L);
    }
}

// row[t0 .. t0+15] as float with 16-byte loads (row + t0 16-byte aligned,
// whole tile in range).
template <typename T>
__device__ __forceinline__ void load16_vec(const T* __restrict__ p, float (&o)[16]) {
    if constexpr (sizeof(T) == 4) {
        const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = q[i];
            o[4 * i] = v.x; o[4 * i + 1] = v.y; o[4 * i + 2] = v.z; o[4 * i + 3] = v.w;
        }
    } else {
        const uint4* q = reinterpret_cast<const uint4*>(p);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint4 v = q[i];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if constexpr (__is_same(T, bf16_t)) {
                    o[8 * i + 2 * k] = __uint_as_float(w[k] << 16);
                    o[8 * i + 2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
                } else {
                    o[8 * i + 2 * k] = float(__builtin_bit_cast(_Float16, uint16_t(w[k] & 0xffffu)));
                    o[8 * i + 2 * k + 1] = float(__builtin_bit_cast(_Float16, uint16_t(w[k] >> 16)));
                }
            }
        }
    }
}

// ---------------------------------------------------- B / C tile staging --
// A 16-state x 16-step tile of B (or C) is staged in LDS as 16-byte chunks:
// chunk i (steps 4i..4i+3 for fp32, 8i..8i+7 for 16-bit types) of state row
// n goes to chunk slot tile_slot(n, i), chosen so that 8 lanes reading chunk
// i of rows 0..7 with ds_read_b128 hit 8 distinct groups of 4 banks.
//   fp32 : 4 chunks per row, slot 4 n + ((i + (n >> 1)) & 3)       (64 slots)
//   16-bit: 2 chunks per row, slot 2 n + ((i + (n >> 2)) & 1)      (32 slots)
template <int kChunksPerRow>
__device__ __forceinline__ int tile_slot(int n, int i) {
    if constexpr (kChunksPerRow == 4) return 4 * n + ((i + (n >> 1)) & 3);
    else return 2 * n + ((i + (n >> 2)) & 1);
}
// Inverse: the (row, chunk) stored in slot p.
template <int kChunksPerRow>
__device__ __forceinline__ void tile_slot_inv(int p, int& n, int& i) {
    if constexpr (kChunksPerRow == 4) { n = p >> 2; i = ((p & 3) - (n >> 1)) & 3; }
    else { n = p >> 1; i = ((p & 1) - (n >> 2)) & 1; }
}

// Eight 16-bit values (bf16 or fp16, 16-byte aligned) as float.
template <typename T>
__device__ __forceinline__ void load8_16(const T* p, float (&o)[8]) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
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

// B / C tile slot of (state n, step t) in a 16-state x 16-step tile.  LDS
// bank model of gfx950 (measured): 4-byte accesses see 32 banks of 4 bytes,
// 8- and 16-byte accesses see 64.  4-step groups are XOR-swizzled by n >> 2,
// so the 16 lanes of states 0..15 reading one group with ds_read_b128 cover
// all 64 banks once, and a staging row of 16 steps (4-byte writes) fills one
// 32-bank half.
__device__ __forceinline__ int bc_slot(int n, int t) { return n * kT + 4 * ((t >> 2) ^ ((n >> 2) & 3)) + (t & 3); }
// Workgroup barrier that orders LDS only.  __syncthreads() also waits for
// every outstanding global load and store of the wave (vmcnt(0)), which
// would drain the loads prefetched for the next tile; the kernels here only
// exchange data through LDS across a barrier.
__device__ __forceinline__ void lds_barrier() {
    __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ------------------------------------------------------- cross-lane ops --
// Value of lane K of this lane's 16-lane row (DPP row_newbcast); folds into
// the consuming VALU instruction as a DPP source modifier.
template <int K>
__device__ __forceinline__ float row_bcast(float v) {
    static_assert(K >= 0 && K < 16, "row lane");
    // every lane of the row is written, so no "old" value is needed (mov_dpp
    // leaves it undefined, which lets the DPP combiner fold the move and
    // avoids a v_mov 0 per broadcast)
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x150 + K, 0xf, 0xf, true));
}

// Row broadcasts fused into the consuming instruction, written as inline asm:
// the compiler folds a row_newbcast move only into a single VOP2 use and
// never into v_fmac_f32, so a broadcast value used twice, or as the
// multiplicand of an accumulation, would otherwise cost a v_mov_b32_dpp per
// lane and step.
//   bmul<K>(s, y)        = s[lane K of the row] * y        (v_mul_f32_dpp)
//   bfmac<K>(acc, s, y) : acc += s[lane K of the row] * y  (v_fmac_f32_dpp)
// Hazards: gfx950 needs two wait states between a VALU write of a VGPR and a
// DPP read of it, and one between a transcendental result and a VALU that
// reads it.  The compiler does not look inside inline asm for either, so
// every broadcast source goes through dpp_sources_ready() after it is
// computed (the asm's outputs are the only definitions the DPP reads see),
// and no transcendental result is passed straight into these helpers.  The
// gfx950 assembly of the library is checked for both rules by the test suite.
template <int K>
__device__ __forceinline__ float bmul(float s, float y) {
    static_assert(K >= 0 && K < 16, "row lane");
    float r;
    __asm__("v_mul_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
            : "=v"(r) : "v"(s), "v"(y), "n"(K));
    return r;
}
template <int K>
__device__ __forceinline__ void bfmac(float& acc, float s, float y) {
    static_assert(K >= 0 && K < 16, "row lane");
    __asm__("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
            : "+v"(acc) : "v"(s), "v"(y), "n"(K));
}
// Two wait states after the last write of the broadcast sources a, b, c.
__device__ __forceinline__ void dpp_sources_ready(float& a, float& b, float& c) {
    __asm__ volatile("s_nop 1" : "+v"(a), "+v"(b), "+v"(c));
}

__device__ __forceinline__ void dpp_sources_ready4(float4& a, float4& b) {
    __asm__ volatile("s_nop 1" : "+v"(a.x), "+v"(a.y), "+v"(a.z), "+v"(a.w), "+v"(b.x), "+v"(b.y), "+v"(b.z), "+v"(b.w));
}

// Value of lane r ^ 8 of this lane's 16-lane row (DPP row_ror:8).
__device__ __forceinline__ float row_ror8(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xf, 0xf, true));
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
// r is sum over the row's lanes r' of v_{r'}[r].  `wbuf` is a per-wave
// scratch of kTrWave floats.  Only lanes of the calling wave touch it and a
// wave executes its LDS operations in order, so no barrier is needed; the
// compiler cannot reorder the accesses because their offsets depend on the
// lane index.  Split in a write and a read so that other work can be placed
// between them.
__device__ __forceinline__ void row_transpose_write(float* wbuf, const float (&v)[16], int j, int r) {
    float* wp = wbuf + j * kTrRow + r * kTrStride;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        *reinterpret_cast<float4*>(wp + 4 * i) = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}
__device__ __forceinline__ float row_transpose_read(const float* wbuf, int j, int r) {
    const float* rp = wbuf + j * kTrRow + r;
    // all 16 reads are issued before the first add (one LDS round trip)
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = rp[k * kTrStride];
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1) {
#pragma unroll
        for (int k = 0; k < w; ++k) v[k] += v[k + w];
    }
    return v[0];
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
// All branch-free: a per-lane branch would make the compiler wait for every
// outstanding load, including the prefetch of the next tile.

// log(1 + e) for e >= 0, accurate for small e: log(u) * e / (u - 1) with
// u = 1 + e rounded (Goldberg's compensation), and e itself when u == 1.
__device__ __forceinline__ float log1p_pos(float e) {
    const float u = 1.f + e;   // in [1, 2]: no denormal or range handling needed
    const float l = (__builtin_amdgcn_logf(u) * 0.69314718055994531f) * __builtin_amdgcn_rcpf(u - 1.f) * e;
    return u == 1.f ? e : l;
}

// softplus with the reference's threshold rule, log1p(exp(x)) for x <= 20
// and x above (forward_kernel.cu:217-221), computed as the identity
// max(x, 0) + log1p(exp(-|x|)); for x > 20 the second term (< 2.1e-9) is
// below half an ulp of x, so the result is exactly x as in the reference.
__device__ __forceinline__ float softplus20(float x) {
    return fmaxf(x, 0.f) + log1p_pos(__expf(-fabsf(x)));
}

// 1 / (1 + exp(-x)); exp overflow gives 1 / inf = 0.
__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

// Workgroups are dispatched round-robin over the XCDs (blockIdx.x % kXcds
// runs on XCD blockIdx.x % kXcds).  This renumbering hands each XCD a
// contiguous range of logical workgroup ids, so the workgroups of one batch
// row, which read the same B / C and add into the same dB / dC, share one
// XCD's L2.  Grids that are not a multiple of kXcds keep the plain order.
__device__ __forceinline__ int64_t xcd_block_id() {
    const uint32_t n = gridDim.x, i = blockIdx.x;
    if (n % kXcds != 0) return i;
    return int64_t(i % kXcds) * (n / kXcds) + i / kXcds;
}

// Global (address space 1) pointers.  Loads, stores and atomics through them
// are global_* instructions even where the compiler cannot infer the address
// space itself; flat_* forms would also count against lgkmcnt, which the
// LDS-only barrier waits on.
#define SS_GLOBAL __attribute__((address_space(1)))

// Builtin vector types for global accesses (the HIP vector classes cannot be
// assigned from address-space-qualified lvalues).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// A workgroup-uniform pointer, as a global pointer pinned to scalar
// registers.  Loop strength reduction otherwise turns base + t0 + offset
// into a 64-bit per-lane induction variable, which costs 64-bit adds per
// access and loses the scalar-base + 32-bit-offset address form.
template <typename T>
__device__ __forceinline__ SS_GLOBAL T* gbase(T* p) {
    SS_GLOBAL T* g = (SS_GLOBAL T*)p;
#if defined(__HIP_DEVICE_COMPILE__)   // register constraints exist only in the gfx950 pass
    __asm__("" : "+s"(g));
#endif
    return g;
}

// p advanced by `bytes`, a 32-bit per-lane offset (callers keep it below
// 2^32: the launchers check the strides that go into it).
// The empty asm keeps the 32-bit offset next to its use: hoisted out of a
// loop, its zero-extension to 64 bits would be materialised there, and the
// access would again be a 64-bit per-lane address.
template <typename T>
__device__ __forceinline__ SS_GLOBAL T* goff(SS_GLOBAL T* p, uint32_t bytes) {
#if defined(__HIP_DEVICE_COMPILE__)
    __asm__("" : "+v"(bytes));
#endif
    return (SS_GLOBAL T*)((SS_GLOBAL char*)p + bytes);
}

// Buffer resources: a workgroup-uniform base held in SGPRs, addressed by a
// 32-bit per-lane byte offset (VGPR) plus a uniform byte offset (SGPR), so
// neither the row base nor the chunk advance costs VALU address arithmetic.
// The launchers check that every offset a kernel forms stays below 2^32, and
// the scan kernels' resources end with their arrays (make_rsrc_in).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;   // gfx9-family raw buffer, 32-bit data format
__device__ __forceinline__ rsrc_t make_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, -1, kRsrcWord3);
}
// As make_rsrc with nrec bytes: -1 for the whole range, or 0 for a resource
// of zero bytes, through which the hardware's range check drops every store
// (and loads return 0), so an optional output costs no branch in the loop
// and no memory traffic.  nrec must be uniform and come from a kernel
// argument: a record count the compiler selects in a VGPR makes every
// access through the resource a waterfall loop.
__device__ __forceinline__ rsrc_t make_rsrc_n(const void* base, int nrec) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nrec, kRsrcWord3);
}
// A resource at byte `off` of an array whose elements end `end` bytes after
// its base pointer: the hardware's range check drops any access past the
// array (loads read 0), and every access when `end` is 0 (an absent optional
// array).  The record count is made wave-uniform so that the resource stays
// in SGPRs (a per-lane count would make every access a waterfall loop).
__device__ __forceinline__ rsrc_t make_rsrc_in(const void* array, int64_t off, int64_t end) {
    const int64_t left = end - off;
    const uint32_t nrec = left <= 0 ? 0u : (left >= int64_t(0xffffffffu) ? 0xffffffffu : uint32_t(left));
    const char* base = array ? static_cast<const char*>(array) + off : nullptr;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), 0,
                                             __builtin_amdgcn_readfirstlane(int(nrec)), kRsrcWord3);
}
// Element (voff + soff bytes) of an IT array as float.
template <typename T>
__device__ __forceinline__ float bload(rsrc_t r, uint32_t voff, uint32_t soff) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, int(voff), int(soff), 0));
    } else {
        const uint32_t v = __builtin_amdgcn_raw_buffer_load_b16(r, int(voff), int(soff), 0);
        if constexpr (__is_same(T, bf16_t)) return __uint_as_float(v << 16);
        else return float(__builtin_bit_cast(_Float16, uint16_t(v)));
    }
}
// Cache policy of a buffer store: kStoreNT marks the data non-temporal
// (the cache keeps it for the shortest time), for streams nothing in the
// same kernel reads again.
constexpr int kStoreDefault = 0, kStoreNT = 2;
template <typename T, int kPolicy = kStoreDefault>
__device__ __forceinline__ void bstore(rsrc_t r, uint32_t voff, uint32_t soff, float v) {
    if constexpr (sizeof(T) == 4) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, int(voff), int(soff), kPolicy);
    } else {
        uint16_t h;
        if constexpr (__is_same(T, bf16_t)) h = io<bf16_t>::round(v);
        else h = __builtin_bit_cast(uint16_t, _Float16(v));
        __builtin_amdgcn_raw_buffer_store_b16(h, r, int(voff), int(soff), kPolicy);
    }
}
// Four consecutive elements (voff + soff bytes, element aligned) as float4:
// one 16-byte (fp32) or 8-byte (16-bit types) access per lane.  The shader
// memory pipeline runs in its unaligned mode under the HSA runtime, so the
// access need not be aligned to its size.
template <typename T>
__device__ __forceinline__ float4 bload4(rsrc_t r, uint32_t voff, uint32_t soff) {
    if constexpr (sizeof(T) == 4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, int(voff), int(soff), 0);
        return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
    } else {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, int(voff), int(soff), 0);
        if constexpr (__is_same(T, bf16_t)) {
            return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                               __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u));
        } else {
            return make_float4(float(__builtin_bit_cast(_Float16, uint16_t(v.x & 0xffffu))),
                               float(__builtin_bit_cast(_Float16, uint16_t(v.x >> 16))),
                               float(__builtin_bit_cast(_Float16, uint16_t(v.y & 0xffffu))),
                               float(__builtin_bit_cast(_Float16, uint16_t(v.y >> 16))));
        }
    }
}
// Stores of more than 8 bytes read their data VGPRs after issue, and a VALU
// write to those VGPRs too soon after the store corrupts the stored data.
// The compiler inserts the wait states for that only when the store's
// uniform offset is not a register, so this store takes no uniform offset:
// callers fold their advance into the resource base.
template <typename T, int kPolicy = kStoreDefault>
__device__ __forceinline__ void bstore4(rsrc_t r, uint32_t voff, float4 v) {
    if constexpr (sizeof(T) == 4) {
        const u32x4 w = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
        __builtin_amdgcn_raw_buffer_store_b128(w, r, int(voff), 0, kPolicy);
    } else if constexpr (__is_same(T, bf16_t)) {
        const u32x2 w = {io<bf16_t>::pack2(v.x, v.y), io<bf16_t>::pack2(v.z, v.w)};
        __builtin_amdgcn_raw_buffer_store_b64(w, r, int(voff), 0, kPolicy);
    } else {
        const u32x2 w = {uint32_t(__builtin_bit_cast(uint16_t, _Float16(v.x))) |
                             (uint32_t(__builtin_bit_cast(uint16_t, _Float16(v.y))) << 16),
                         uint32_t(__builtin_bit_cast(uint16_t, _Float16(v.z))) |
                             (uint32_t(__builtin_bit_cast(uint16_t, _Float16(v.w))) << 16)};
        __builtin_amdgcn_raw_buffer_store_b64(w, r, int(voff), 0, kPolicy);
    }
}
__device__ __forceinline__ float f4get(const float4& v, int c) { return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w; }

// fp32 atomic add through a buffer resource (no return value).
__device__ __forceinline__ void batomic_add(rsrc_t r, uint32_t voff, uint32_t soff, float v) {
    __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(v, r, int(voff), int(soff), 0);
}

// fp32 atomic add to LDS (ds_add_f32, no return value).
__device__ __forceinline__ void lds_add(float* p, float v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// fp32 atomic add through a global pointer (no return value).
__device__ __forceinline__ void gatomic_add(SS_GLOBAL float* p, float v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace ss
