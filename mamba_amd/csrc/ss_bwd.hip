// Backward selective scan for gfx950.
//
// Gradients follow the reference backward kernel
// (csrc/selective_scan/backward_kernel.cu:276-585), with g the adjoint of h:
//   g_t = a_{t+1} g_{t+1} + dy_t C_t              (reverse scan, :386-431)
//   du_t = D dy_t + delta'_t sum_n g B            (:334,437-438)
//   ddelta'_t = u_t sum_n g B + sum_n A g a_t h_{t-1}   (:439-440)
//   dA += delta' g a_t h_{t-1}   dB += g delta' u   dC += dy h_t   (:441-454)
//   dD += dy u; ddelta = ddelta' sigmoid(delta + bias) below 20; dbias += ddelta
// and, for the fused z gate, dy = dout silu(z), dz = dout y silu'(z) with the
// pre-gate output y saved by the forward.
//
// Same lane layout as the forward: a lane owns one (channel, state) chain.
// Chunks of kChunk steps are visited last to first.  For each chunk the lane
// restarts the forward recurrence from the checkpoint the forward stored in
// x, keeps a_t and h_t of the chunk in registers, then runs the adjoint
// backwards over the chunk.  Per-step partial values are streamed to LDS four
// steps at a time:
//  - sums over states (sum_n g B, sum_n A g a h) are in-row transposed sums;
//  - sums over channels (dB, dC) are summed over the workgroup's 16 channels
//    and added to global memory once per workgroup and (state, step).
#include "ss_device.hpp"
#include "ss_kernels.hpp"

namespace ss {

static_assert(kChunk == kT, "the backward walks one 16-step tile per checkpoint chunk");

// LDS layouts (gfx950 LDS serves 32 banks of 4 bytes; a float4 write is
// served 8 lanes at a time, a dword read 32 lanes at a time).
//
// Per-wave transposition buffers for the sums over states: [row j][lane r]
// [step k], 256 floats per row, rows 272 floats apart (so odd rows start 16
// banks over).  The four steps 4c..4c+3 of lane r are stored as a float4 at
// chunk slot c ^ ((r >> 1) & 3), so 8 consecutive lanes write 8 distinct
// bank groups and the two rows read by one dword read hit disjoint bank
// halves.
constexpr int kTrRowStride = kT * kT + 16;                      // 272 floats
constexpr int kTrArr = (kRows - 1) * kTrRowStride + kT * kT;    // 1072 floats
__device__ __forceinline__ int tr_row(int j) { return j * kTrRowStride; }
__device__ __forceinline__ int tr_pos(int r, int c4) { return r * kT + 4 * (c4 ^ ((r >> 1) & 3)); }
// Workgroup buffer for the sums over channels: [channel][state][step] with
// the same per-(state) swizzle; 16 x 256 floats per array.
constexpr int kChArr = kChPerWG * kT * kT;     // 4096 floats

// kVarBC: B and C are both variable (the common case, no runtime switches).
template <typename IT, int SPL, bool kVarBC>
__global__ __launch_bounds__(kThreads, 2) void ss_bwd_kernel(const BwdParams q) {
    __shared__ __attribute__((aligned(16))) float trb[kWaves * 2 * kTrArr];   // [wave][s1, s2]
    __shared__ __attribute__((aligned(16))) float chb[2 * kChArr];           // [dB, dC]
    const FwdParams& p = q.f;

    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int r = lane & 15;
    const int j = lane >> 4;
    const int64_t nblk = (p.dim + kChPerWG - 1) / kChPerWG;
    const int64_t blk = xcd_block_id();
    const int64_t b = blk / nblk;
    const int64_t c_raw = (blk % nblk) * kChPerWG + w * kRows + j;
    const bool cval = c_raw < p.dim;
    const int64_t c = cval ? c_raw : p.dim - 1;
    const int64_t g = c / p.dpg;
    const int N = int(p.dstate);
    const int64_t L = p.seqlen;
    const bool var_B = kVarBC || p.var_B;
    const bool var_C = kVarBC || p.var_C;

    float* tr_s1 = trb + (w * 2 + 0) * kTrArr + tr_row(j);
    float* tr_s2 = trb + (w * 2 + 1) * kTrArr + tr_row(j);
    float* ch_dB = chb + (w * kRows + j) * kT * kT;
    float* ch_dC = chb + kChArr + (w * kRows + j) * kT * kT;
    // in-row transposed sum: element (lane r', step r) of the row lives at
    // r' * 16 + 4 * ((r >> 2) ^ ((r' >> 1) & 3)) + (r & 3) from the row base
    int toff[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) toff[m] = 4 * ((r >> 2) ^ m) + (r & 3);

    const IT* u = static_cast<const IT*>(p.u) + b * p.u_bs + c * p.u_ds;
    const IT* dl = static_cast<const IT*>(p.delta) + b * p.dl_bs + c * p.dl_ds;
    // without a z gate zp / yp alias u so that their (unused) loads stay unconditional
    const IT* zp = p.has_z ? static_cast<const IT*>(p.z) + b * p.z_bs + c * p.z_ds : u;
    const IT* yp = p.has_z ? static_cast<const IT*>(p.y) + b * p.y_bs + c * p.y_ds : u;
    const IT* dop = static_cast<const IT*>(q.dout) + b * q.do_bs + c * q.do_ds;
    IT* dup = static_cast<IT*>(q.du) + b * q.du_bs + c * q.du_ds;
    IT* ddp = static_cast<IT*>(q.ddelta) + b * q.dd_bs + c * q.dd_ds;
    IT* dzp = p.has_z ? static_cast<IT*>(q.dz) + b * q.dz_bs + c * q.dz_ds : nullptr;
    const IT* Bv_base = static_cast<const IT*>(p.B) + b * p.B_bs + g * p.B_gs;
    const IT* Cv_base = static_cast<const IT*>(p.C) + b * p.C_bs + g * p.C_gs;
    const float* Bc_base = static_cast<const float*>(p.B) + c * p.B_gs;
    const float* Cc_base = static_cast<const float*>(p.C) + c * p.C_gs;
    // x: (batch, chunk, dim, dstate)
    const float* xrow = p.x + (b * p.n_chunks * p.dim + c) * N;
    const int64_t x_chunk_stride = p.dim * N;
    // fp32 gradient rows of variable B / C for this (batch, group): (dstate, seqlen)
    const int64_t G = p.dim / p.dpg;
    float* dBrow = q.dB + (b * G + g) * int64_t(N) * L;
    float* dCrow = q.dC + (b * G + g) * int64_t(N) * L;

    const float Dv = p.D ? p.D[c] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[c] : 0.f;
    const bool pad_states = (N % 16) != 0;

    float A2[SPL], Av[SPL], Bc[SPL], Cc[SPL];
    float gcar[SPL], acar[SPL], dA_acc[SPL], dBc_acc[SPL], dCc_acc[SPL];
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
        const int n = 16 * s + r;
        const bool nv = n < N;
        Av[s] = nv ? p.A[c * p.A_ds + n * p.A_ns] : 0.f;
        A2[s] = Av[s] * kLog2e;
        Bc[s] = (!var_B && nv) ? Bc_base[n * p.B_ns] : 0.f;
        Cc[s] = (!var_C && nv) ? Cc_base[n * p.C_ns] : 0.f;
        gcar[s] = 0.f;      // g_{t+1} entering the chunk from the right
        acar[s] = 1.f;      // a_{t+1} entering the chunk from the right
        dA_acc[s] = 0.f;
        dBc_acc[s] = 0.f;
        dCc_acc[s] = 0.f;
    }
    float dD_acc = 0.f, db_acc = 0.f;

    // B / C rows of state group s for the chunk at t0; padding states get
    // C = 0 so that their adjoint g stays 0.
    auto load_bc = [&](int64_t t0, int s, float (&Bo)[kT], float (&Co)[kT]) {
        const int n = 16 * s + r;
        const bool nv = n < N;
        const int nn = nv ? n : N - 1;
        if (var_B) load_tile16<IT>(Bv_base + nn * p.B_ns, t0, L, p.vec_B != 0, Bo);
        else {
#pragma unroll
            for (int k = 0; k < kT; ++k) Bo[k] = Bc[s];
        }
        if (var_C) load_tile16<IT>(Cv_base + nn * p.C_ns, t0, L, p.vec_C != 0, Co);
        else {
#pragma unroll
            for (int k = 0; k < kT; ++k) Co[k] = Cc[s];
        }
        if (pad_states && !nv) {
#pragma unroll
            for (int k = 0; k < kT; ++k) Co[k] = 0.f;
        }
    };
    // checkpoint h at the end of chunk ck - 1 (0 before the first chunk)
    auto load_h0 = [&](int64_t ck, int s) {
        const int n = 16 * s + r;
        const int nn = n < N ? n : N - 1;
        const float v = xrow[(ck > 0 ? ck - 1 : 0) * x_chunk_stride + nn];
        return ck > 0 ? v : 0.f;
    };

    // Per-step inputs of step 16 ck + r (streams from HBM), loaded two chunks
    // ahead and shifted along; chunk indices below 0 re-read chunk 0.
    struct Step { float u, dl, dout, z, y; };
    auto load_step = [&](int64_t ck, Step& S) {
        const int64_t t = (ck >= 0 ? ck : 0) * kT + r;
        if (t - r + kT <= L) {
            S.u = load_at(u, t); S.dl = load_at(dl, t); S.dout = load_at(dop, t);
            S.z = load_at(zp, t); S.y = load_at(yp, t);
        } else {
            S.u = load_or0(u, t, L); S.dl = load_or0(dl, t, L); S.dout = load_or0(dop, t, L);
            S.z = load_or0(zp, t, L); S.y = load_or0(yp, t, L);
        }
    };
    // B / C rows and checkpoint of the chunk (single state group), one chunk ahead.
    struct Rows { float h0; float B[kT], C[kT]; };
    auto load_rows = [&](int64_t ck, Rows& R) {
        if constexpr (SPL == 1) {
            const int64_t ckc = ck >= 0 ? ck : 0;
            load_bc(ckc * kT, 0, R.B, R.C);
            R.h0 = load_h0(ckc, 0);
        }
    };

    auto compute_chunk = [&](int64_t ck, const Step& S, Rows& R) {
        const int64_t t0 = ck * kT;
        const int64_t t = t0 + r;
        const bool tv = t < L;
        const int nval = int(L - t0 < kT ? L - t0 : kT);
        const float pre = S.dl + bias;
        float dt = p.softplus ? softplus20(pre) : pre;
        if (!tv) dt = 0.f;
        const float dtu = dt * S.u;
        const float sgz = sigmoidf_(S.z);
        float dy = p.has_z ? S.dout * S.z * sgz : S.dout;
        if (!cval) dy = 0.f;     // padding channels contribute nothing
        float s1_red = 0.f, s2_red = 0.f;

#pragma unroll
        for (int s = 0; s < SPL; ++s) {
            const int n = 16 * s + r;
            const bool nv = n < N;
            float Bl[kT], Cl[kT];
            float h0 = 0.f;
            if constexpr (SPL > 1) {
                load_bc(t0, s, Bl, Cl);
                h0 = load_h0(ck, s);
            } else {
                h0 = R.h0;
            }
            const float (&Bt)[kT] = (SPL == 1) ? R.B : Bl;
            const float (&Ct)[kT] = (SPL == 1) ? R.C : Cl;

            // ---- recompute a_t and h_t of the chunk from the checkpoint
            float as[kT], hs[kT];
            float hcur = h0;
            const float a2 = A2[s];
            static_for<kT>([&](auto K) {
                constexpr int k = decltype(K)::value;
                const float a = __builtin_amdgcn_exp2f(row_bcast<k>(dt) * a2);
                hcur = __builtin_fmaf(a, hcur, row_bcast<k>(dtu) * Bt[k]);
                as[k] = a;
                hs[k] = hcur;
            });

            // ---- adjoint, last step of the chunk first, streamed to LDS four steps at a time
            float gv = gcar[s];
            float anext = acar[s];
            const float av = Av[s];
            float dAq = 0.f, dBq = 0.f, dCq = 0.f;
            static_for<4>([&](auto KG) {
                constexpr int kg = 3 - decltype(KG)::value;
                float s1p[4], s2p[4], dBp[4], dCp[4];
                static_for<4>([&](auto KI) {
                    constexpr int ki = 3 - decltype(KI)::value;
                    constexpr int k = 4 * kg + ki;
                    const float dyk = row_bcast<k>(dy);
                    gv = __builtin_fmaf(anext, gv, dyk * Ct[k]);
                    float hprev;
                    if constexpr (k == 0) hprev = h0;
                    else hprev = hs[k - 1];
                    const float gah = gv * (as[k] * hprev);
                    dAq = __builtin_fmaf(row_bcast<k>(dt), gah, dAq);
                    s2p[ki] = av * gah;
                    s1p[ki] = gv * Bt[k];
                    dBp[ki] = gv * row_bcast<k>(dtu);
                    dCp[ki] = dyk * hs[k];
                    anext = as[k];
                });
                const int o = tr_pos(r, kg);
                *reinterpret_cast<float4*>(tr_s1 + o) = make_float4(s1p[0], s1p[1], s1p[2], s1p[3]);
                *reinterpret_cast<float4*>(tr_s2 + o) = make_float4(s2p[0], s2p[1], s2p[2], s2p[3]);
                if (var_B) {
                    if (q.wg_reduce) {
                        *reinterpret_cast<float4*>(ch_dB + o) = make_float4(dBp[0], dBp[1], dBp[2], dBp[3]);
                    } else if (cval && nv) {
#pragma unroll
                        for (int ki = 0; ki < 4; ++ki)
                            if (4 * kg + ki < nval) atomicAdd(dBrow + n * L + t0 + 4 * kg + ki, dBp[ki]);
                    }
                } else {
                    dBq += (dBp[0] + dBp[1]) + (dBp[2] + dBp[3]);
                }
                if (var_C) {
                    if (q.wg_reduce) {
                        *reinterpret_cast<float4*>(ch_dC + o) = make_float4(dCp[0], dCp[1], dCp[2], dCp[3]);
                    } else if (cval && nv) {
#pragma unroll
                        for (int ki = 0; ki < 4; ++ki)
                            if (4 * kg + ki < nval) atomicAdd(dCrow + n * L + t0 + 4 * kg + ki, dCp[ki]);
                    }
                } else {
                    dCq += (dCp[0] + dCp[1]) + (dCp[2] + dCp[3]);
                }
            });
            gcar[s] = gv;
            acar[s] = anext;
            dA_acc[s] += dAq;
            dBc_acc[s] += dBq;
            dCc_acc[s] += dCq;

            // in-row transposed sums over states
            float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
            for (int rr = 0; rr < kT; rr += 2) {
                a0 += tr_s1[toff[(rr >> 1) & 3] + rr * kT];
                a1 += tr_s1[toff[((rr + 1) >> 1) & 3] + (rr + 1) * kT];
                b0 += tr_s2[toff[(rr >> 1) & 3] + rr * kT];
                b1 += tr_s2[toff[((rr + 1) >> 1) & 3] + (rr + 1) * kT];
            }
            s1_red += a0 + a1;
            s2_red += b0 + b1;

            // sums over the workgroup's 16 channels, one global add per (state, step)
            if (q.wg_reduce && (var_B || var_C)) {
                __syncthreads();
                const int tid = threadIdx.x;
                const int nl = tid >> 4, k = tid & 15;
                const int ridx = nl * kT + 4 * ((k >> 2) ^ ((nl >> 1) & 3)) + (k & 3);
                const int ng = 16 * s + nl;
#pragma unroll
                for (int arr = 0; arr < 2; ++arr) {
                    const bool use = arr == 0 ? var_B : var_C;
                    if (!use) continue;
                    const float* src = chb + arr * kChArr + ridx;
                    float s0 = 0.f, s1 = 0.f;
#pragma unroll
                    for (int ch = 0; ch < kChPerWG; ch += 2) {
                        s0 += src[ch * kT * kT];
                        s1 += src[(ch + 1) * kT * kT];
                    }
                    float* dst = arr == 0 ? dBrow : dCrow;
                    if (ng < N && k < nval) atomicAdd(dst + ng * L + t0 + k, s0 + s1);
                }
                __syncthreads();
            }
        }

        // ---- per-step outputs of step t0 + r
        const float du = Dv * dy + dt * s1_red;
        const float ddt = S.u * s1_red + s2_red;
        const float dd = p.softplus ? ddt * sigmoidf_(pre) : ddt;
        if (tv && cval) {
            io<IT>::store(dup + t, du);
            io<IT>::store(ddp + t, dd);
            if (p.has_z) io<IT>::store(dzp + t, S.dout * S.y * sgz * (1.f + S.z * (1.f - sgz)));
            dD_acc += dy * S.u;
            db_acc += dd;
        }
    };

    // per-step inputs: three chunks in flight (shifted by register moves);
    // B / C rows: two buffers alternated by unrolling the chunk loop twice
    const int64_t nck = p.n_chunks;
    Step S0, S1, S2;
    Rows R0, R1;
    load_step(nck - 1, S0);
    load_step(nck - 2, S1);
    load_rows(nck - 1, R0);
    for (int64_t ck = nck - 1; ck >= 0; ck -= 2) {
        load_step(ck - 2, S2);
        load_rows(ck - 1, R1);
        compute_chunk(ck, S0, R0);
        S0 = S1; S1 = S2;
        load_step(ck - 3, S2);
        load_rows(ck - 2, R0);
        if (ck - 1 >= 0) compute_chunk(ck - 1, S0, R1);
        S0 = S1; S1 = S2;
    }

    // ---- per-channel and per-(channel, state) sums over time and batch
    dD_acc = row_allsum(dD_acc);
    db_acc = row_allsum(db_acc);
    if (cval && r == 0) {
        if (q.dD) atomicAdd(q.dD + c, dD_acc);
        if (q.ddelta_bias) atomicAdd(q.ddelta_bias + c, db_acc);
    }
    if (cval) {
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
            const int n = 16 * s + r;
            if (n < N) {
                atomicAdd(q.dA + c * N + n, dA_acc[s]);
                if (!var_B) atomicAdd(q.dB + c * N + n, dBc_acc[s]);
                if (!var_C) atomicAdd(q.dC + c * N + n, dCc_acc[s]);
            }
        }
    }
}

// ------------------------------------------------------------ fast path --
// dstate 16, variable B and C, seqlen a multiple of 32, dim and channels per
// group multiples of 16, z gate fixed at compile time: no branch around a
// memory access in the loop (see the forward fast path).  Global traffic is
// workgroup-cooperative per 32-step super-tile (two checkpoint chunks):
// every thread moves one 2-element piece of each of u, delta, dout, z, y, B
// and C, prefetched one super-tile ahead and staged in LDS; du, ddelta and
// dz go back the same way.  The sums over states (sum_n g B, sum_n A g a h)
// share one float2 transposition per chunk.  dB / dC are first summed over
// the wave's 4 channel rows with v_permlane32_swap / v_permlane16_swap, then
// over the 4 waves in LDS once per super-tile (inside barriers the
// super-tile needs anyway), and added to global memory once per workgroup,
// state and step.
constexpr int kSB = 32;                 // steps per backward super-tile
constexpr int kQB = kSB / kT;           // chunks per super-tile
constexpr int kStrB = kSB + 16;         // LDS row stride of stream tiles (floats)
constexpr int kWgN = kSB + 1;           // padded step stride of the dB / dC wave partials
constexpr int kBCB = kSB + 4;           // LDS row stride of B / C tiles (floats)
constexpr int kTrHRow = kT * 16;        // half-chunk (s1, s2) transposition: 16 lanes x 8 steps x 2 (256 floats)

template <typename IT>
struct Piece2 {                         // 2 consecutive elements of one row
    using raw = typename std::conditional<sizeof(IT) == 4, u32x2, uint32_t>::type;
    raw v;
    __device__ __forceinline__ void load(const SS_GLOBAL IT* p) { v = *(const SS_GLOBAL raw*)p; }
    __device__ __forceinline__ float2 f() const {
        if constexpr (sizeof(IT) == 4) {
            return make_float2(__uint_as_float(v.x), __uint_as_float(v.y));
        } else if constexpr (__is_same(IT, bf16_t)) {
            return make_float2(__uint_as_float(v << 16), __uint_as_float(v & 0xffff0000u));
        } else {
            return make_float2(float(__builtin_bit_cast(_Float16, uint16_t(v & 0xffffu))),
                               float(__builtin_bit_cast(_Float16, uint16_t(v >> 16))));
        }
    }
};

template <typename IT>
__device__ __forceinline__ void store2(SS_GLOBAL IT* p, float2 v) {
    if constexpr (sizeof(IT) == 4) {
        *(SS_GLOBAL f32x2*)p = f32x2{v.x, v.y};
    } else if constexpr (__is_same(IT, bf16_t)) {
        *(SS_GLOBAL uint32_t*)p = io<bf16_t>::pack2(v.x, v.y);
    } else {
        *(SS_GLOBAL uint32_t*)p = uint32_t(__builtin_bit_cast(uint16_t, _Float16(v.x))) |
                                  (uint32_t(__builtin_bit_cast(uint16_t, _Float16(v.y))) << 16);
    }
}

// Sum of v0..v3 (steps 4kg + 0..3 of one state) over the wave's 4 rows; row
// j of the result holds the sum for step 4kg + j.
__device__ __forceinline__ float rows4_sum(float v0, float v1, float v2, float v3) {
    auto s02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v0), __float_as_uint(v2), false, false);
    auto s13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v1), __float_as_uint(v3), false, false);
    // rows 0, 1: steps 0 / 1 over rows {j, j + 2}; rows 2, 3: steps 2 / 3
    const float a = __uint_as_float(s02[0]) + __uint_as_float(s02[1]);
    const float c = __uint_as_float(s13[0]) + __uint_as_float(s13[1]);
    auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(c), false, false);
    return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}

template <typename IT, bool kZ>
// 3 workgroups per CU (12 waves): at most 168 VGPRs and 54,272 B of LDS
// (LDS float atomics would save space but are far slower than this layout).
__global__ __launch_bounds__(kThreads, 3) void ss_bwd_fast(const BwdParams q) {
    // streams u, delta, dout, z, y; the first three hold du, ddelta, dz afterwards
    __shared__ __attribute__((aligned(16))) float s_in[5 * kChPerWG * kStrB];
    __shared__ __attribute__((aligned(16))) float s_B[16 * kBCB];
    __shared__ __attribute__((aligned(16))) float s_C[16 * kBCB];
    __shared__ __attribute__((aligned(16))) float s_tr[kWaves * kRows * kTrHRow];   // [wave][row][lane][8 steps][2]
    __shared__ __attribute__((aligned(16))) float s_wg[2 * kWaves * 16 * kWgN];     // [dB, dC][wave][n][t]
    const FwdParams& p = q.f;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int r = lane & 15;
    const int j = lane >> 4;
    const int row = w * kRows + j;
    const int64_t nblk = p.dim / kChPerWG;
    const int64_t blk = xcd_block_id();
    const int64_t b = blk / nblk;
    const int64_t c0 = (blk % nblk) * kChPerWG;
    const int64_t c = c0 + row;
    const int64_t g = c0 / p.dpg;
    const int64_t L = p.seqlen;
    const int64_t G = p.dim / p.dpg;

    // cooperative piece of this thread: row prow, steps 2 pc, 2 pc + 1.
    // Workgroup-uniform bases plus 32-bit per-thread offsets.
    const int prow = tid >> 4, pc = tid & 15;
    const IT* bu = static_cast<const IT*>(p.u) + b * p.u_bs + c0 * p.u_ds;
    const IT* bd = static_cast<const IT*>(p.delta) + b * p.dl_bs + c0 * p.dl_ds;
    const IT* bo = static_cast<const IT*>(q.dout) + b * q.do_bs + c0 * q.do_ds;
    const IT* bz = kZ ? static_cast<const IT*>(p.z) + b * p.z_bs + c0 * p.z_ds : bu;
    const IT* by = kZ ? static_cast<const IT*>(p.y) + b * p.y_bs + c0 * p.y_ds : bu;
    const IT* bB = static_cast<const IT*>(p.B) + b * p.B_bs + g * p.B_gs;
    const IT* bC = static_cast<const IT*>(p.C) + b * p.C_bs + g * p.C_gs;
    IT* bdu = static_cast<IT*>(q.du) + b * q.du_bs + c0 * q.du_ds;
    IT* bdd = static_cast<IT*>(q.ddelta) + b * q.dd_bs + c0 * q.dd_ds;
    IT* bdz = kZ ? static_cast<IT*>(q.dz) + b * q.dz_bs + c0 * q.dz_ds : bdu;
    // per-thread byte offsets (below 2^32, checked by bwd_fast_ok)
    constexpr uint32_t es = sizeof(IT);
    const uint32_t ou = uint32_t(prow * p.u_ds + 2 * pc) * es, od = uint32_t(prow * p.dl_ds + 2 * pc) * es;
    const uint32_t oo = uint32_t(prow * q.do_ds + 2 * pc) * es;
    const uint32_t oz = kZ ? uint32_t(prow * p.z_ds + 2 * pc) * es : ou;
    const uint32_t oy = kZ ? uint32_t(prow * p.y_ds + 2 * pc) * es : ou;
    const uint32_t oB = uint32_t(prow * p.B_ns + 2 * pc) * es, oC = uint32_t(prow * p.C_ns + 2 * pc) * es;
    const uint32_t odu = uint32_t(prow * q.du_ds + 2 * pc) * es, odd = uint32_t(prow * q.dd_ds + 2 * pc) * es;
    const uint32_t odz = kZ ? uint32_t(prow * q.dz_ds + 2 * pc) * es : odu;
    const int spos = prow * kStrB + 2 * pc;
    const int bpos = prow * kBCB + 2 * pc;
    // x: (batch, chunk, dim, dstate); the checkpoint of this lane's chain
    const float* gx = p.x + (b * p.n_chunks * p.dim + c0) * kT;
    const uint32_t ox = uint32_t(row * kT + r) * 4u;
    const int64_t x_chunk_stride = p.dim * kT;
    // dB / dC of this batch row and group, or of its slice of the workspace
    const int64_t slice = (c0 / kChPerWG) % q.ws_slices;
    float* dBb = (q.ws ? q.ws + 2 * slice * q.ws_stride : q.dB) + (b * G + g) * int64_t(kT) * L;
    float* dCb = (q.ws ? q.ws + (2 * slice + 1) * q.ws_stride : q.dC) + (b * G + g) * int64_t(kT) * L;

    const float Dv = p.D ? p.D[c] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[c] : 0.f;
    const float av = p.A[c * p.A_ds + r * p.A_ns];
    const float a2 = av * kLog2e;
    const bool softplus = p.softplus != 0;

    // (s1, s2) summed over the row's 16 states, 8 steps (half a chunk) at a
    // time: lane n stores steps 2m, 2m+1 of the half (m = 0..3) as a float4 at
    // n * 16 + 4 * (m ^ ((n >> 1) & 3)); lane r then adds states
    // n = 2 i + (r >> 3) (i = 0..7) of step r & 7, and the other 8 states come
    // from lane r ^ 8 (DPP row_ror:8).  Both access patterns are free of bank
    // conflicts.
    float* trw = s_tr + (w * kRows + j) * kTrHRow;

    struct Pieces {
        Piece2<IT> u, d, o, z, y, B, C;
        float x[kQB];
    };
    auto fetch = [&](int64_t st, Pieces& P) {     // st clamped by the caller
        const int64_t t0 = st * kSB;
        P.u.load(goff(gbase(bu + t0), ou));
        P.d.load(goff(gbase(bd + t0), od));
        P.o.load(goff(gbase(bo + t0), oo));
        if constexpr (kZ) { P.z.load(goff(gbase(bz + t0), oz)); P.y.load(goff(gbase(by + t0), oy)); }
        P.B.load(goff(gbase(bB + t0), oB));
        P.C.load(goff(gbase(bC + t0), oC));
#pragma unroll
        for (int qq = 0; qq < kQB; ++qq) {
            const int64_t ck = st * kQB + qq;
            const float v = *goff(gbase(gx + (ck > 0 ? ck - 1 : 0) * x_chunk_stride), ox);
            P.x[qq] = ck > 0 ? v : 0.f;
        }
    };
    auto stage = [&](const Pieces& P) {
        constexpr int T = kChPerWG * kStrB;
        *reinterpret_cast<float2*>(s_in + 0 * T + spos) = P.u.f();
        *reinterpret_cast<float2*>(s_in + 1 * T + spos) = P.d.f();
        *reinterpret_cast<float2*>(s_in + 2 * T + spos) = P.o.f();
        if constexpr (kZ) {
            *reinterpret_cast<float2*>(s_in + 3 * T + spos) = P.z.f();
            *reinterpret_cast<float2*>(s_in + 4 * T + spos) = P.y.f();
        }
        *reinterpret_cast<float2*>(s_B + bpos) = P.B.f();
        *reinterpret_cast<float2*>(s_C + bpos) = P.C.f();
    };
    // dB / dC of the super-tile at t0: sum the 4 wave partials; thread tid adds
    // steps 2 (tid & 15), +1 of state tid >> 4
    auto flush_dbc = [&](int64_t t0) {
        const int nl = tid >> 4, k = 2 * (tid & 15);
        float sB0 = 0.f, sB1 = 0.f, sC0 = 0.f, sC1 = 0.f;
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) {
            const float* pb = s_wg + ((0 * kWaves + ww) * 16 + nl) * kWgN + k;
            const float* pcc = s_wg + ((1 * kWaves + ww) * 16 + nl) * kWgN + k;
            sB0 += pb[0]; sB1 += pb[1]; sC0 += pcc[0]; sC1 += pcc[1];
        }
        const uint32_t o = uint32_t(nl * L + k) * 4u;
        gatomic_add(goff(gbase(dBb + t0), o), sB0);
        gatomic_add(goff(gbase(dBb + t0 + 1), o), sB1);
        gatomic_add(goff(gbase(dCb + t0), o), sC0);
        gatomic_add(goff(gbase(dCb + t0 + 1), o), sC1);
    };

    float gacar = 0.f, dA_acc = 0.f, dD_acc = 0.f, db_acc = 0.f;
    const int64_t nst = L / kSB;
    Pieces P;
    fetch(nst - 1, P);
    for (int64_t st = nst - 1; st >= 0; --st) {
        const int64_t t0 = st * kSB;
        lds_barrier();                 // previous super-tile's outputs and dB / dC partials are consumed
        stage(P);
        float h0s[kQB];
#pragma unroll
        for (int qq = 0; qq < kQB; ++qq) h0s[qq] = P.x[qq];
        lds_barrier();
        fetch(st > 0 ? st - 1 : 0, P);              // prefetch the previous super-tile

        float in_v[5][kQB];
#pragma unroll
        for (int a = 0; a < 5; ++a)
#pragma unroll
            for (int qq = 0; qq < kQB; ++qq)
                in_v[a][qq] = (a < 3 || kZ) ? s_in[a * kChPerWG * kStrB + row * kStrB + kT * qq + r] : 0.f;
        lds_barrier();                 // s_in is reused for the outputs below

#pragma unroll
        for (int qi = kQB - 1; qi >= 0; --qi) {
            const float uu = in_v[0][qi], pre = in_v[1][qi] + bias, dout = in_v[2][qi];
            const float zz = in_v[3][qi], yv = in_v[4][qi];
            float dt = softplus ? softplus20(pre) : pre;
            float dtu = dt * uu;
            const float sgz = kZ ? sigmoidf_(zz) : 1.f;
            float dy = kZ ? dout * zz * sgz : dout;
            dpp_sources_ready(dt, dtu, dy);
            const float h0 = h0s[qi];
            const float* sBr = s_B + r * kBCB + kT * qi;
            const float* sCr = s_C + r * kBCB + kT * qi;

            // ---- recompute a_t and h_t of the chunk from the checkpoint
            float as[kT], hs[kT];
            static_for<kT>([&](auto K) {
                constexpr int k = decltype(K)::value;
                // the compiler's own fused broadcast: it knows the consumer is a
                // transcendental and needs no wait state after a plain VALU
                as[k] = __builtin_amdgcn_exp2f(row_bcast<k>(dt) * a2);
            });
            float hcur = h0;
            static_for<4>([&](auto I) {
                constexpr int i = decltype(I)::value;
                const float4 vb = *reinterpret_cast<const float4*>(sBr + 4 * i);
                const float bq[4] = {vb.x, vb.y, vb.z, vb.w};
                static_for<4>([&](auto KI) {
                    constexpr int k = 4 * i + decltype(KI)::value;
                    hcur = __builtin_fmaf(as[k], hcur, bmul<k>(dtu, bq[k & 3]));
                    hs[k] = hcur;
                });
            });

            // ---- adjoint, last step first, four steps at a time; s1r / s2r get
            // this lane's step r of the sums over states.  ga carries
            // g_{t+1} a_{t+1}: it is both the decayed adjoint entering step t
            // and, times h_{t-1}, the dA / ddelta term of step t + 1.
            float ga = gacar;
            float s1r = 0.f, s2r = 0.f;
            static_for<4>([&](auto KG) {
                constexpr int kg = 3 - decltype(KG)::value;
                const float4 vb = *reinterpret_cast<const float4*>(sBr + 4 * kg);
                const float4 vc = *reinterpret_cast<const float4*>(sCr + 4 * kg);
                const float bq[4] = {vb.x, vb.y, vb.z, vb.w};
                const float cq[4] = {vc.x, vc.y, vc.z, vc.w};
                float s1p[4], s2p[4], dBp[4], dCp[4];
                static_for<4>([&](auto KI) {
                    constexpr int ki = 3 - decltype(KI)::value;
                    constexpr int k = 4 * kg + ki;
                    float gv = ga;
                    bfmac<k>(gv, dy, cq[ki]);            // g_t = a_{t+1} g_{t+1} + dy_t C_t
                    ga = gv * as[k];
                    float hprev;
                    if constexpr (k == 0) hprev = h0;
                    else hprev = hs[k - 1];
                    const float gah = ga * hprev;        // g_t a_t h_{t-1}
                    bfmac<k>(dA_acc, dt, gah);
                    s2p[ki] = av * gah;
                    s1p[ki] = gv * bq[ki];
                    dBp[ki] = bmul<k>(dtu, gv);
                    dCp[ki] = bmul<k>(dy, hs[k]);
                });
                // (s1, s2) of steps 4kg..4kg+3 as two float4 (steps 2m, 2m+1 of the half)
                *reinterpret_cast<float4*>(trw + r * 16 + 4 * ((2 * (kg & 1)) ^ ((r >> 1) & 3))) =
                    make_float4(s1p[0], s2p[0], s1p[1], s2p[1]);
                *reinterpret_cast<float4*>(trw + r * 16 + 4 * ((2 * (kg & 1) + 1) ^ ((r >> 1) & 3))) =
                    make_float4(s1p[2], s2p[2], s1p[3], s2p[3]);
                // dB / dC of steps 4kg..4kg+3 summed over the wave's rows:
                // row j holds step 4kg + j
                const float dBs = rows4_sum(dBp[0], dBp[1], dBp[2], dBp[3]);
                const float dCs = rows4_sum(dCp[0], dCp[1], dCp[2], dCp[3]);
                s_wg[((0 * kWaves + w) * 16 + r) * kWgN + kT * qi + 4 * kg + j] = dBs;
                s_wg[((1 * kWaves + w) * 16 + r) * kWgN + kT * qi + 4 * kg + j] = dCs;
                if constexpr ((kg & 1) == 0) {   // half kg / 2 is complete: sum it
                    constexpr int h = kg >> 1;
                    const int e = r & 1, m = (r & 7) >> 1, nh = r >> 3;
                    float2 v[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const int n = 2 * i + nh;
                        v[i] = *reinterpret_cast<const float2*>(trw + n * 16 + 4 * (m ^ ((n >> 1) & 3)) + 2 * e);
                    }
#pragma unroll
                    for (int wdt = 4; wdt >= 1; wdt >>= 1)
#pragma unroll
                        for (int i = 0; i < wdt; ++i) { v[i].x += v[i + wdt].x; v[i].y += v[i + wdt].y; }
                    const float t1 = v[0].x + row_ror8(v[0].x);
                    const float t2 = v[0].y + row_ror8(v[0].y);
                    if (nh == h) { s1r = t1; s2r = t2; }
                }
            });
            gacar = ga;


            // ---- per-step outputs of step t0 + 16 qi + r into the output tiles
            const float du = Dv * dy + dt * s1r;
            const float ddt = uu * s1r + s2r;
            const float dd = softplus ? ddt * sigmoidf_(pre) : ddt;
            const int opos = row * kStrB + kT * qi + r;
            s_in[0 * kChPerWG * kStrB + opos] = du;
            s_in[1 * kChPerWG * kStrB + opos] = dd;
            if constexpr (kZ) s_in[2 * kChPerWG * kStrB + opos] = dout * yv * sgz * (1.f + zz * (1.f - sgz));
            dD_acc += dy * uu;
            db_acc += dd;
        }
        lds_barrier();
        flush_dbc(t0);
        constexpr int T = kChPerWG * kStrB;
        store2<IT>(goff(gbase(bdu + t0), odu), *reinterpret_cast<const float2*>(s_in + 0 * T + spos));
        store2<IT>(goff(gbase(bdd + t0), odd), *reinterpret_cast<const float2*>(s_in + 1 * T + spos));
        if constexpr (kZ) store2<IT>(goff(gbase(bdz + t0), odz), *reinterpret_cast<const float2*>(s_in + 2 * T + spos));
    }

    // ---- per-channel and per-(channel, state) sums over time and batch
    dD_acc = row_allsum(dD_acc);
    db_acc = row_allsum(db_acc);
    if (r == 0) {
        if (q.dD) atomicAdd(q.dD + c, dD_acc);
        if (q.ddelta_bias) atomicAdd(q.ddelta_bias + c, db_acc);
    }
    atomicAdd(q.dA + c * kT + r, dA_acc);
}

bool bwd_fast_ok(const BwdParams& q) {
    const FwdParams& p = q.f;
    return p.dstate == 16 && p.var_B && p.var_C && p.seqlen >= kSB && p.seqlen % kSB == 0 &&
           p.dim % kChPerWG == 0 && p.dpg % kChPerWG == 0 && p.stream_vec && q.stream_vec_bwd &&
           (!p.has_z || p.y != nullptr) &&
           small_strides({p.seqlen, p.u_ds, p.dl_ds, p.z_ds, p.y_ds, p.B_ns, p.C_ns,
                          q.do_ds, q.du_ds, q.dd_ds, q.dz_ds});
}

// ------------------------------------------------------- dB / dC slices --
// Clears up to kZeroSegs float arrays in one launch: the workspace slices
// and, when the caller asks for it, the gradient accumulators.  A fill
// kernel rather than memsets, so the whole backward can be captured in a
// graph.
struct ZeroSegs {
    float* p[kZeroSegs];
    int64_t n[kZeroSegs];
    int count;
};

__global__ __launch_bounds__(256) void ss_zero_segs(const ZeroSegs z) {
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    for (int s = 0; s < z.count; ++s) {
        float* p = z.p[s];
        const int64_t n = z.n[s];
        int64_t head = 0;
        if ((reinterpret_cast<uintptr_t>(p) & 15) == 0) {
            const int64_t n4 = n >> 2;
            float4* p4 = reinterpret_cast<float4*>(p);
            for (int64_t i = tid; i < n4; i += stride) p4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            head = 4 * n4;
        }
        for (int64_t i = head + tid; i < n; i += stride) p[i] = 0.f;
    }
}

// dB (+)= sum of the dB slices, dC (+)= sum of the dC slices (n4 float4
// each); `overwrite` ignores what dB / dC held.
__global__ __launch_bounds__(256) void ss_ws_reduce(const float4* __restrict__ ws, int slices, int64_t n4,
                                                    float4* __restrict__ dB, float4* __restrict__ dC,
                                                    int overwrite) {
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
        float4 sb = overwrite ? make_float4(0.f, 0.f, 0.f, 0.f) : dB[i];
        float4 sc = overwrite ? make_float4(0.f, 0.f, 0.f, 0.f) : dC[i];
        for (int k = 0; k < slices; ++k) {
            const float4 vb = ws[(2 * k) * n4 + i], vc = ws[(2 * k + 1) * n4 + i];
            sb.x += vb.x; sb.y += vb.y; sb.z += vb.z; sb.w += vb.w;
            sc.x += vc.x; sc.y += vc.y; sc.z += vc.z; sc.w += vc.w;
        }
        dB[i] = sb;
        dC[i] = sc;
    }
}

// Launches the clearing pass for p: workspace slices, and with zero_grads
// the accumulators (dB / dC only when no slice sum overwrites them).
static hipError_t launch_zero(const BwdParams& p, bool sliced, hipStream_t stream) {
    ZeroSegs z{};
    int64_t most = 0;
    auto add = [&](float* ptr, int64_t n) {
        if (!ptr || n <= 0) return;
        z.p[z.count] = ptr;
        z.n[z.count] = n;
        ++z.count;
        most = n > most ? n : most;
    };
    if (sliced) add(p.ws, 2 * p.ws_slices * p.ws_stride);
    if (p.zero_grads) {
        add(p.dA, p.dA_n);
        add(p.dD, p.dD_n);
        add(p.ddelta_bias, p.dD_n);
        if (!sliced) {
            add(p.dB, p.dB_n);
            add(p.dC, p.dC_n);
        }
    }
    if (z.count == 0) return hipSuccess;
    const int64_t blocks = (most / 4 + 255) / 256;
    const unsigned grid = unsigned(blocks < 1 ? 1 : (blocks > 2048 ? 2048 : blocks));
    hipLaunchKernelGGL(ss_zero_segs, dim3(grid), dim3(256), 0, stream, z);
    return hipGetLastError();
}

hipError_t launch_bwd_zero_only(const BwdParams& p, hipStream_t stream) { return launch_zero(p, false, stream); }

int bwd_ws_slices(const BwdParams& p) {
    if (!bwd_fast_ok(p)) return 1;
    // about 12 channel blocks per slice; a handful of slices already removes
    // most of the contention, more only cost reduction traffic
    const int64_t blocks = p.f.dpg / kChPerWG;
    const int64_t k = (blocks + 11) / 12;
    return int(k < 1 ? 1 : (k > 16 ? 16 : k));
}

template <typename IT>
static hipError_t launch_bwd_t(const BwdParams& p, hipStream_t stream) {
    const int64_t nblk = (p.f.dim + kChPerWG - 1) / kChPerWG;
    const dim3 grid(unsigned(nblk * p.f.batch));
    const dim3 block(kThreads);
    const int spl = int((p.f.dstate + 15) / 16);
    const bool vbc = p.f.var_B && p.f.var_C;
    const bool fast = bwd_fast_ok(p);
    const bool sliced = fast && p.ws != nullptr;
    hipError_t e = launch_zero(p, sliced, stream);
    if (e != hipSuccess) return e;
    if (fast) {
        const int64_t n4 = sliced ? p.ws_stride / 4 : 0;
        const unsigned rgrid = unsigned(n4 > 0 ? (n4 + 255) / 256 < 2048 ? (n4 + 255) / 256 : 2048 : 1);
        if (p.f.has_z) hipLaunchKernelGGL((ss_bwd_fast<IT, true>), grid, block, 0, stream, p);
        else hipLaunchKernelGGL((ss_bwd_fast<IT, false>), grid, block, 0, stream, p);
        if (sliced) {
            hipLaunchKernelGGL(ss_ws_reduce, dim3(rgrid), dim3(256), 0, stream,
                               reinterpret_cast<const float4*>(p.ws), int(p.ws_slices), n4,
                               reinterpret_cast<float4*>(p.dB), reinterpret_cast<float4*>(p.dC),
                               int(p.zero_grads));
        }
    } else if (spl <= 1) {
        if (vbc) hipLaunchKernelGGL((ss_bwd_kernel<IT, 1, true>), grid, block, 0, stream, p);
        else hipLaunchKernelGGL((ss_bwd_kernel<IT, 1, false>), grid, block, 0, stream, p);
    } else if (spl <= 2) hipLaunchKernelGGL((ss_bwd_kernel<IT, 2, false>), grid, block, 0, stream, p);
    else if (spl <= 4) hipLaunchKernelGGL((ss_bwd_kernel<IT, 4, false>), grid, block, 0, stream, p);
    else if (spl <= 8) hipLaunchKernelGGL((ss_bwd_kernel<IT, 8, false>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((ss_bwd_kernel<IT, 16, false>), grid, block, 0, stream, p);
    return hipGetLastError();
}

const char* bwd_kernel_name(const BwdParams& p) { return bwd_fast_ok(p) ? "ss_bwd_fast" : "ss_bwd_kernel"; }

hipError_t launch_bwd(const BwdParams& p, int itype, hipStream_t stream) {
    switch (itype) {
        case SS_F32: return launch_bwd_t<float>(p, stream);
        case SS_BF16: return launch_bwd_t<bf16_t>(p, stream);
        case SS_F16: return launch_bwd_t<_Float16>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace ss
