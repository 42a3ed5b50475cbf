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
    // the workgroup's first channel: dB / dC are summed over its 16 channels
    // in LDS, one run of channels per group, and added once per (state,
    // step) and group (channels past dim count as the last one: they add
    // exact zeros)
    const int64_t wc0 = (blk % nblk) * kChPerWG;
    // bit ch: channel ch is the last of its group in the workgroup (uniform:
    // kept in a scalar register, so the branches on it are scalar)
    uint32_t run_end_v = 1u << (kChPerWG - 1);
    for (int ch = 0; ch < kChPerWG - 1; ++ch) {
        const int64_t nc = wc0 + ch + 1;
        if (nc < p.dim && nc % p.dpg == 0) run_end_v |= 1u << ch;
    }
    const uint32_t run_end = __builtin_amdgcn_readfirstlane(run_end_v);
    const bool one_group = run_end == 1u << (kChPerWG - 1);
    const int64_t g0 = wc0 / p.dpg;
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
    // fp32 gradient rows of variable B / C: (batch, group, dstate, seqlen)
    const int64_t G = p.dim / p.dpg;

    const float Dv = p.D ? p.D[c] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[c] : 0.f;
    // lanes past dstate: the last group's past dstate % 16, or whole groups
    // when dstate is below 16 SPL (48 on SPL 4)
    const bool pad_states = N < 16 * SPL;

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
                    *reinterpret_cast<float4*>(ch_dB + o) = make_float4(dBp[0], dBp[1], dBp[2], dBp[3]);
                } else {
                    dBq += (dBp[0] + dBp[1]) + (dBp[2] + dBp[3]);
                }
                if (var_C) {
                    *reinterpret_cast<float4*>(ch_dC + o) = make_float4(dCp[0], dCp[1], dCp[2], dCp[3]);
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

            // sums over the workgroup's 16 channels, one global add per (state,
            // step) and group of them
            if (var_B || var_C) {
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
                    float* dst = (arr == 0 ? q.dB : q.dC) + (int64_t(ng) * L + t0 + k);
                    const bool add = ng < N && k < nval;
                    if (one_group) {
                        float s0 = 0.f, s1 = 0.f;
#pragma unroll
                        for (int ch = 0; ch < kChPerWG; ch += 2) {
                            s0 += src[ch * kT * kT];
                            s1 += src[(ch + 1) * kT * kT];
                        }
                        if (add) atomicAdd(dst + (b * G + g0) * int64_t(N) * L, s0 + s1);
                    } else {
                        float sum = 0.f;
                        int64_t gc = g0;
#pragma unroll
                        for (int ch = 0; ch < kChPerWG; ++ch) {
                            sum += src[ch * kT * kT];
                            if ((run_end >> ch) & 1u) {
                                if (add) atomicAdd(dst + (b * G + gc) * int64_t(N) * L, sum);
                                sum = 0.f;
                                ++gc;
                            }
                        }
                    }
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
// dstate 16, variable B and C, seqlen a multiple of 16, dim and channels per
// group multiples of 16, z gate fixed at compile time: no branch around a
// memory access in the loop (on gfx950 the compiler waits for every
// outstanding load at a branch, which would serialise the prefetch).
//
// One 16-step chunk per iteration, last chunk first, one barrier per chunk:
//  - per-step inputs (u, delta, dout, z, y) and the checkpoint come straight
//    from HBM into the lane that owns the step (a row's 16 lanes read one
//    64-byte segment), two chunks ahead; du, ddelta, dz go back the same way;
//  - the B / C tile of the chunk (shared by the workgroup's 16 channels) is
//    staged through LDS, double-buffered, one chunk ahead;
//  - sums over states (sum_n g B, sum_n A g a h) use a per-row LDS
//    transposition with one region per half chunk, so the reads of one half
//    overlap the arithmetic of the next; A_n is applied inside that sum;
//  - dB / dC: summed over the wave's 4 rows with v_permlane32_swap /
//    v_permlane16_swap, over the 4 waves through LDS (double-buffered), and
//    added to global memory once per workgroup, state and step, one chunk
//    later (after the next barrier).
constexpr int kTrHRow = kT * 16;        // half-chunk (s1, s2) transposition: 16 lanes x 8 steps x 2 (256 floats)
constexpr int kTrRowB = kTrHRow + 32;   // per-row region, padded so rows j, j + 1 use different 64-bank halves

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

// dB / dC wave-partial slot of (step t, state n): state XOR-swizzled by step,
// conflict-free both for rows writing (4 steps x 16 states) and for the
// flush reading (16 steps x 2 states).
__device__ __forceinline__ int wg_slot(int t, int n) { return t * 16 + (n ^ t); }

// kDet: deterministic sums (plain stores of the partials, summed in a fixed
// order afterwards) instead of atomic adds.
// kAcc: one pass of a state-sliced backward (dstate 16 S, one pass per
// 16-state slice): the sums over states of each step (sum_n g B, sum_n A g a h)
// are added to those of the earlier slices (p.acc, fp32) and, but in the last
// pass, stored back there; the per-step outputs computed from them are only
// kept in the last pass (the host sets the other passes' extents to 0).
// kVB / kVC: B / C vary per step (tile through LDS, dB / dC per (state,
// step) summed over the workgroup's channels and added to global memory);
// false: constant, (dim, dstate) fp32, held in registers, with dB / dC per
// (channel, state) accumulated in each lane over the chunks and added once
// at the end.  With both constant the kernel has no B / C tile, no dB / dC
// flush and no barrier.
template <typename IT, bool kZ, bool kDet, bool kAcc, bool kVB, bool kVC>
// 3 workgroups per CU (12 waves): at most 168 VGPRs and about 53 KB of LDS
// (3 x 53,248 B share a CU; at 54,272 B only 2 do, measured).
__global__ __launch_bounds__(kThreads, 3) void ss_bwd_fast(const BwdParams q) {
    __shared__ __attribute__((aligned(16))) float s_bc[2 * 2 * 16 * kT];              // [buf][B, C][n][t]
    __shared__ __attribute__((aligned(16))) float s_tr[kWaves * kRows * kTrRowB];     // [wave][row][lane][8 steps][2]
    __shared__ __attribute__((aligned(16))) float s_wg[2 * 2 * kWaves * kT * 16];     // [buf][dB, dC][wave][t][n]
    const FwdParams& p = q.f;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int r = lane & 15;
    const int j = lane >> 4;
    const int row = w * kRows + j;
    const int64_t nblk = p.dim / kChPerWG;
    // logical workgroup (b, seg, channel block), channel block fastest
    const int64_t blk = xcd_block_id();
    const int nseg = p.nseg;
    const int64_t bs = blk / nblk;
    const int64_t b = bs / nseg;
    const int seg = int(bs % nseg);
    const int64_t c0 = (blk % nblk) * kChPerWG;
    const int64_t c = c0 + row;
    const int64_t g = c0 / p.dpg;
    const int64_t L = p.seqlen;
    const int64_t G = p.dim / p.dpg;
    // chunks of 16 steps, padded to an even count: a ragged seqlen ends in a
    // partial chunk and, for an odd count, one wholly past the sequence; both
    // are the first two this kernel runs (the tail), made of identity steps
    const int nck = int((L + 2 * kT - 1) / (2 * kT)) * 2;   // below 2^22 (seqlen < 2^26)
    // this workgroup's chunks [k0, k1), an even number starting at an even index
    const int k0 = 2 * seg_begin(seg, nck / 2, nseg), k1 = 2 * seg_begin(seg + 1, nck / 2, nseg);

    // Buffer resources at the workgroup's rows; lane (row, r) owns step r of
    // channel c0 + row and, for the B / C staging, step r of state row.  The
    // chunk advance is the uniform offset.  Offsets stay below 2^32 (checked
    // by bwd_fast_ok).
    constexpr int64_t es64 = sizeof(IT);
    const rsrc_t Ru = make_rsrc_in(p.u, (b * p.u_bs + c0 * p.u_ds) * es64, p.u_end);
    const rsrc_t Rd = make_rsrc_in(p.delta, (b * p.dl_bs + c0 * p.dl_ds) * es64, p.dl_end);
    const rsrc_t Ro = make_rsrc_in(q.dout, (b * q.do_bs + c0 * q.do_ds) * es64, q.do_end);
    const rsrc_t Rz = kZ ? make_rsrc_in(p.z, (b * p.z_bs + c0 * p.z_ds) * es64, p.z_end) : make_rsrc_n(nullptr, 0);
    const rsrc_t Ry = kZ ? make_rsrc_in(p.y, (b * p.y_bs + c0 * p.y_ds) * es64, p.y_end) : make_rsrc_n(nullptr, 0);
    const rsrc_t RB = kVB ? make_rsrc_in(p.B, (b * p.B_bs + g * p.B_gs) * es64, p.B_end) : make_rsrc_n(nullptr, 0);
    const rsrc_t RC = kVC ? make_rsrc_in(p.C, (b * p.C_bs + g * p.C_gs) * es64, p.C_end) : make_rsrc_n(nullptr, 0);
    const rsrc_t Rdu = make_rsrc_in(q.du, (b * q.du_bs + c0 * q.du_ds) * es64, q.du_end);
    const rsrc_t Rdd = make_rsrc_in(q.ddelta, (b * q.dd_bs + c0 * q.dd_ds) * es64, q.dd_end);
    const rsrc_t Rdz = kZ ? make_rsrc_in(q.dz, (b * q.dz_bs + c0 * q.dz_ds) * es64, q.dz_end) : make_rsrc_n(nullptr, 0);
    // dB / dC of this batch row and group, or of its slice of the workspace
    // (rows of ld floats)
    const int64_t slice = (c0 / kChPerWG) % q.ws_slices;
    const int64_t ld = q.bc_ld;
    const int64_t bc_off = (b * G + g) * (kAcc ? q.bc_N : int64_t(kT)) * ld * 4;
    const rsrc_t RdB = q.ws ? make_rsrc_in(q.ws, 2 * slice * q.ws_stride * 4 + bc_off, q.ws_end)
                            : make_rsrc_in(q.dB, bc_off, q.dB_end);
    const rsrc_t RdC = q.ws ? make_rsrc_in(q.ws, (2 * slice + 1) * q.ws_stride * 4 + bc_off, q.ws_end)
                            : make_rsrc_in(q.dC, bc_off, q.dC_end);
    constexpr uint32_t es = sizeof(IT);
    const uint32_t ou = uint32_t(row * p.u_ds + r) * es, od = uint32_t(row * p.dl_ds + r) * es;
    const uint32_t oo = uint32_t(row * q.do_ds + r) * es;
    const uint32_t oz = uint32_t(row * p.z_ds + r) * es, oy = uint32_t(row * p.y_ds + r) * es;
    const uint32_t oB = uint32_t(row * p.B_ns + r) * es, oC = uint32_t(row * p.C_ns + r) * es;
    const uint32_t odu = uint32_t(row * q.du_ds + r) * es, odd = uint32_t(row * q.dd_ds + r) * es;
    const uint32_t odz = uint32_t(row * q.dz_ds + r) * es;
    // x: (batch, chunk, dim, xN), 16 unless the call is state-sliced
    const int64_t xN = kAcc ? p.xN : kT;
    const uint32_t ox = uint32_t(row * xN + r) * 4u;
    // x: (batch, chunk, dim, dstate); the checkpoint of this lane's chain,
    // through a resource based at a window of chunks whose offsets stay below
    // p.x_win (2^31 bytes unless the caller set a smaller span; offsets from
    // the row's first chunk would pass 2^32 once
    // seqlen x dim reaches 2^30); the chunks run last to first, and a window
    // is rebased (to end at the chunk) when a chunk leaves it, which at most
    // rows never happens
    const int64_t x_off = (b * p.n_chunks * p.dim + c0) * xN * 4;
    const int64_t x_chunk_bytes = p.dim * xN * 4;
    const int x_wck = int(p.x_win / x_chunk_bytes) > 0 ? int(p.x_win / x_chunk_bytes) : 1;
    int x_w0 = k1 - x_wck > 0 ? k1 - x_wck : 0;
    rsrc_t Rx = make_rsrc_in(p.x, x_off + int64_t(x_w0) * x_chunk_bytes, p.x_end);
    auto x_load = [&](int ckx) {
        if (ckx < x_w0) {
            x_w0 = ckx - x_wck + 1 > 0 ? ckx - x_wck + 1 : 0;
            Rx = make_rsrc_in(p.x, x_off + int64_t(x_w0) * x_chunk_bytes, p.x_end);
        }
        return bload<float>(Rx, ox, uint32_t(ckx - x_w0) * uint32_t(x_chunk_bytes));
    };

    const float Dv = p.D ? p.D[c] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[c] : 0.f;
    const float a2 = p.A[c * p.A_ds + r * p.A_ns] * kLog2e;
    const bool softplus = p.softplus != 0;
    // constant B / C: this lane's B[c][r], C[c][r], and its dB, dC sums
    const float bconst = kVB ? 0.f : static_cast<const float*>(p.B)[c * p.B_gs + r * p.B_ns];
    const float cconst = kVC ? 0.f : static_cast<const float*>(p.C)[c * p.C_gs + r * p.C_ns];
    float dBc = 0.f, dCc = 0.f;

    // (s1, s2) summed over the row's 16 states, 8 steps (half a chunk) at a
    // time: lane n stores steps 2m, 2m+1 of the half (m = 0..3) as a float4 at
    // n * 16 + 4 * (m ^ (n >> 2)); lane r then adds states n = 2 i + (r >> 3)
    // (i = 0..7) of step r & 7, and the other 8 states come from lane r ^ 8
    // (DPP row_ror:8).  The float4 writes and float2 reads of a wave both take
    // the minimum number of LDS cycles.  One region per row serves both halves:
    // a wave's LDS operations execute in order, so the second half's writes
    // cannot overtake the first half's reads.  s2 is summed with the weights
    // A_n of those states.
    float* trw = s_tr + (w * kRows + j) * kTrRowB;
    const int te = r & 1, tm = (r & 7) >> 1, tnh = r >> 3;
    float Aw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) Aw[i] = p.A[c * p.A_ds + (2 * i + tnh) * p.A_ns];

    // state slices (kAcc): the earlier slices' sums over states of this row's
    // steps, fp32 (batch, dim, seqlen), sum_n g B at p.acc and sum_n A g a h
    // a further batch x dim x seqlen floats on (below 2^31 bytes, checked by
    // the host); read at the start of the step's chunk (a chunk's work
    // covers their latency), stored back (but in the last pass) with its
    // outputs
    const int64_t acc_off = (b * p.dim + c0) * L * 4;
    const uint32_t acc2 = uint32_t(p.batch * p.dim * L * 4);
    const uint32_t oacc = uint32_t(row * L + r) * 4u;
    const rsrc_t Rai = kAcc ? make_rsrc_in(p.acc, acc_off, p.acc_in_end) : make_rsrc_n(nullptr, 0);
    const rsrc_t Rao = kAcc ? make_rsrc_in(p.acc, acc_off, p.acc_out_end) : make_rsrc_n(nullptr, 0);

    struct Chunk { float u, d, o, z, y, B, C, x; };
    auto fetch = [&](int ck, Chunk& P) {     // 0 <= ck < nck
        const uint32_t so = uint32_t(ck * kT) * es;
        P.u = bload<IT>(Ru, ou, so);
        P.d = bload<IT>(Rd, od, so);
        P.o = bload<IT>(Ro, oo, so);
        if constexpr (kZ) {
            P.z = bload<IT>(Rz, oz, so);
            P.y = bload<IT>(Ry, oy, so);
        } else {
            P.z = 0.f;
            P.y = 0.f;
        }
        P.B = kVB ? bload<IT>(RB, oB, so) : 0.f;
        P.C = kVC ? bload<IT>(RC, oC, so) : 0.f;
        const float v = x_load(ck > 0 ? ck - 1 : 0);
        P.x = ck > 0 ? v : 0.f;
    };
    // A chunk of the tail: loads at steps clamped to the sequence, and past
    // its end the inputs of an identity step (delta' = 0, so decay 1 and no
    // input; dout, u, B, C zero), as the reference pads its last chunk
    // (backward_kernel.cu:291-315 with forward_kernel.cu:267-271).
    auto fetch_tail = [&](int ck, Chunk& P) {
        const int t = ck * kT + r;
        const bool in = t < L;
        const int te = in ? t : int(L) - 1;
        P.u = in ? bload<IT>(Ru, uint32_t(row * p.u_ds + te) * es, 0) : 0.f;
        P.d = in ? bload<IT>(Rd, uint32_t(row * p.dl_ds + te) * es, 0) : (softplus ? -INFINITY : -bias);
        P.o = in ? bload<IT>(Ro, uint32_t(row * q.do_ds + te) * es, 0) : 0.f;
        if constexpr (kZ) {
            P.z = in ? bload<IT>(Rz, uint32_t(row * p.z_ds + te) * es, 0) : 0.f;
            P.y = in ? bload<IT>(Ry, uint32_t(row * p.y_ds + te) * es, 0) : 0.f;
        } else {
            P.z = 0.f;
            P.y = 0.f;
        }
        P.B = (kVB && in) ? bload<IT>(RB, uint32_t(row * p.B_ns + te) * es, 0) : 0.f;
        P.C = (kVC && in) ? bload<IT>(RC, uint32_t(row * p.C_ns + te) * es, 0) : 0.f;
        const float v = x_load(ck > 0 ? ck - 1 : 0);
        P.x = ck > 0 ? v : 0.f;
    };
    // this lane's element of the B / C tile (state row, step r) into buffer buf
    auto stage = [&](const Chunk& P, int buf) {
        if constexpr (kVB) s_bc[(buf * 2 + 0) * 16 * kT + bc_slot(row, r)] = P.B;
        if constexpr (kVC) s_bc[(buf * 2 + 1) * 16 * kT + bc_slot(row, r)] = P.C;
    };
    // dB / dC of chunk ck from wave-partial buffer buf: thread (n, t) sums the
    // 4 waves and adds once into global memory (16 consecutive steps per state)
    const int fn = tid >> 4, ft = tid & 15;
    const uint32_t ofl0 = uint32_t(fn * ld + ft) * 4u;
    // split in the LDS reads and the sums + global adds, so that other work
    // can sit between them
    auto flush_read = [&](int buf, float (&v)[2 * kWaves]) {
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) {
            v[ww] = s_wg[((buf * 2 + 0) * kWaves + ww) * kT * 16 + wg_slot(ft, fn)];
            v[kWaves + ww] = s_wg[((buf * 2 + 1) * kWaves + ww) * kT * 16 + wg_slot(ft, fn)];
        }
    };
    // (TAIL: the sums of steps past the sequence are zero, but for a state
    // that is not finite (0 * inf), so they are replaced by exact zeros.  The
    // workspace's padded rows have slots for those steps.  In rows of seqlen
    // floats, which only a call without workspace uses for a ragged seqlen,
    // their zeros go elsewhere: a partial chunk's onto the last step; a chunk
    // wholly past the sequence adds them onto the previous chunk's 16 steps,
    // one per address (onto one address, all workgroups' adds of the chunk
    // were serialised in the atomic unit: seqlen 2064 fp32 took 570 us
    // against 338 us at 2048), where the ones past the sequence land on the
    // first steps of the next state row, or past dB / dC's end, where the
    // resource drops them.  Adding an exact zero changes no value.)
    auto flush_commit = [&](int ck, const float (&v)[2 * kWaves], auto TAIL) {
        float sB = (v[0] + v[1]) + (v[2] + v[3]);
        float sC = (v[4] + v[5]) + (v[6] + v[7]);
        uint32_t so = uint32_t(ck * kT) * 4u;
        uint32_t ofl = ofl0;
        if constexpr (decltype(TAIL)::value) {
            const int t = ck * kT + ft;
            const bool past = t >= L;
            sB = past ? 0.f : sB;
            sC = past ? 0.f : sC;
            if (ck * kT >= ld) {
                so = uint32_t((ck - 1) * kT) * 4u;
            } else if (t >= ld) {
                ofl = uint32_t(fn * ld + int(L) - 1 - ck * kT) * 4u;
            }
        }
        if constexpr (kDet) {
            bstore<float>(RdB, ofl, so, sB);
            bstore<float>(RdC, ofl, so, sC);
        } else {
            if constexpr (kVB) batomic_add(RdB, ofl, so, sB);
            if constexpr (kVC) batomic_add(RdC, ofl, so, sC);
        }
    };
    auto flush = [&](int ck, int buf) {
        if constexpr (!kVB && !kVC) return;
        float v[2 * kWaves];
        flush_read(buf, v);
        flush_commit(ck, v, std::false_type{});
    };

    // the adjoint carry entering this segment from the right: the later
    // segments' carries (each from a zero start) joined right to left,
    // carry <- exp(A sum delta') carry + G
    float gacar = 0.f, dA_acc = 0.f, dD_acc = 0.f, db_acc = 0.f;
    for (int s2 = nseg - 1; s2 > seg; --s2) {
        const int64_t si = (b * nseg + s2) * p.dim + c;
        gacar = __builtin_fmaf(__builtin_amdgcn_exp2f(a2 * p.seg_s[si]), gacar, p.seg_h[si * kT + r]);
    }

    // One chunk: `cur` holds its inputs (fetched two chunks ago) and is
    // refilled with chunk ck - 2; `nxt` holds chunk ck - 1, staged at the end.
    // BUF = ck & 1 is a compile-time constant of each unrolled half, so every
    // LDS address is an immediate offset.
    // TAIL: the chunks that may hold steps past the sequence (the first four
    // run), whose outputs there are dropped.
    auto chunk = [&](int ck_in, Chunk& cur_in, const Chunk& nxt, auto BUF, auto TAIL) {
        constexpr int buf = decltype(BUF)::value;
        constexpr bool kTail = decltype(TAIL)::value;
        // uniform: keeps the chunk's offsets in SGPRs (the tail's masked stores
        // would otherwise turn them into waterfall loops)
        const int ck = __builtin_amdgcn_readfirstlane(ck_in);
        // B / C tile of ck staged; dB / dC partials of ck + 1 complete (the
        // transposition area is per row)
        if constexpr (kVB || kVC) lds_barrier();
        const Chunk cur = cur_in;
        fetch(ck > k0 + 1 ? ck - 2 : k0, cur_in);
        // the earlier slices' sums of this chunk's steps (state slices; the
        // steps past the sequence, in the tail, read 0 through a clamped step)
        float acc1 = 0.f, acc2v = 0.f;
        if constexpr (kAcc) {
            const int t = ck * kT + r;
            const bool tin = !kTail || t < L;
            const uint32_t oa = kTail ? uint32_t(row * L + (tin ? t : int(L) - 1)) * 4u : oacc;
            const uint32_t sa = kTail ? 0u : uint32_t(ck * kT) * 4u;
            const float v1 = bload<float>(Rai, oa, sa), v2 = bload<float>(Rai, oa, sa + acc2);
            acc1 = tin ? v1 : 0.f;
            acc2v = tin ? v2 : 0.f;
        }

        // B / C of this lane's state for the 16 steps of the chunk
        float Bq[kT], Cq[kT];
        const float* sB = s_bc + (buf * 2 + 0) * 16 * kT;
        const float* sC = s_bc + (buf * 2 + 1) * 16 * kT;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (kVB) {
                const float4 vb = *reinterpret_cast<const float4*>(sB + bc_slot(r, 4 * i));
                Bq[4 * i] = vb.x; Bq[4 * i + 1] = vb.y; Bq[4 * i + 2] = vb.z; Bq[4 * i + 3] = vb.w;
            } else {
                Bq[4 * i] = Bq[4 * i + 1] = Bq[4 * i + 2] = Bq[4 * i + 3] = bconst;
            }
            if constexpr (kVC) {
                const float4 vc = *reinterpret_cast<const float4*>(sC + bc_slot(r, 4 * i));
                Cq[4 * i] = vc.x; Cq[4 * i + 1] = vc.y; Cq[4 * i + 2] = vc.z; Cq[4 * i + 3] = vc.w;
            } else {
                Cq[4 * i] = Cq[4 * i + 1] = Cq[4 * i + 2] = Cq[4 * i + 3] = cconst;
            }
        }
        float fv[2 * kWaves];
        if constexpr (kVB || kVC) flush_read(buf ^ 1, fv);

        const float uu = cur.u, pre = cur.d + bias, dout = cur.o, zz = cur.z, yv = cur.y, h0 = cur.x;
        float dt = softplus ? softplus20(pre) : pre;
        float dtu = dt * uu;
        const float sgz = kZ ? sigmoidf_(zz) : 1.f;
        float dy = kZ ? dout * zz * sgz : dout;
        dpp_sources_ready(dt, dtu, dy);

        // ---- recompute a_t and h_t of the chunk from the checkpoint
        float as[kT], hs[kT];
        static_for<kT>([&](auto K) {
            constexpr int k = decltype(K)::value;
            // the compiler's own fused broadcast: it knows the consumer is a
            // transcendental and needs no wait state after a plain VALU
            as[k] = __builtin_amdgcn_exp2f(row_bcast<k>(dt) * a2);
        });
        // the LDS reads issued above have had the decay factors to land
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (kVB || kVC) flush_commit(ck + 1 < k1 ? ck + 1 : k1 - 1, fv, TAIL);
        float hcur = h0;
        static_for<kT>([&](auto K) {
            constexpr int k = decltype(K)::value;
            hcur = __builtin_fmaf(as[k], hcur, bmul<k>(dtu, Bq[k]));
            hs[k] = hcur;
        });

        // the adjoint at raised wave priority: a wave in its dependent chain
        // issues ahead of the SIMD's waves at the chunk start (barrier, LDS
        // reads, decay factors), which wait on memory anyway (measured: fp32
        // 338-342 -> 331-335 us, bf16 batch 4 x dim 5120 x seqlen 8192
        // 2,211-2,278 -> 2,131-2,194 us, same bits)
        __builtin_amdgcn_s_setprio(1);
        // ---- adjoint, last step first, four steps at a time.  ga carries
        // g_{t+1} a_{t+1}: it is both the decayed adjoint entering step t
        // and, times h_{t-1}, the dA / ddelta term of step t + 1.
        float ga = gacar;
        float2 tv1[8], tv0[8];
        float* wgB = s_wg + ((buf * 2 + 0) * kWaves + w) * kT * 16;
        float* wgC = s_wg + ((buf * 2 + 1) * kWaves + w) * kT * 16;
        static_for<4>([&](auto KG) {
            constexpr int kg = 3 - decltype(KG)::value;
            constexpr int hh = kg >> 1;
            float s1p[4], s2p[4], dBp[4], dCp[4];
            static_for<4>([&](auto KI) {
                constexpr int ki = 3 - decltype(KI)::value;
                constexpr int k = 4 * kg + ki;
                float gv = ga;
                bfmac<k>(gv, dy, Cq[k]);             // g_t = a_{t+1} g_{t+1} + dy_t C_t
                ga = gv * as[k];
                float hprev;
                if constexpr (k == 0) hprev = h0;
                else hprev = hs[k - 1];
                const float gah = ga * hprev;        // g_t a_t h_{t-1}
                bfmac<k>(dA_acc, dt, gah);
                s2p[ki] = gah;                       // times A_n in the sum over states
                s1p[ki] = gv * Bq[k];
                // constant B / C: this lane's dB, dC over the steps (a step
                // past the sequence adds nothing, also for a state that is
                // not finite)
                if constexpr (kVB) dBp[ki] = bmul<k>(dtu, gv);
                else if (!kTail || ck * kT + k < L) bfmac<k>(dBc, dtu, gv);
                if constexpr (kVC) dCp[ki] = bmul<k>(dy, hs[k]);
                else if (!kTail || ck * kT + k < L) bfmac<k>(dCc, dy, hs[k]);
            });
            // (s1, s2) of steps 4kg..4kg+3 as two float4 (steps 2m, 2m+1 of the half)
            float* trh = trw;
            *reinterpret_cast<float4*>(trh + r * 16 + 4 * ((2 * (kg & 1)) ^ (r >> 2))) =
                make_float4(s1p[0], s2p[0], s1p[1], s2p[1]);
            *reinterpret_cast<float4*>(trh + r * 16 + 4 * ((2 * (kg & 1) + 1) ^ (r >> 2))) =
                make_float4(s1p[2], s2p[2], s1p[3], s2p[3]);
            // dB / dC of steps 4kg..4kg+3 summed over the wave's rows: row j
            // holds step 4kg + j
            if constexpr (kVB) wgB[wg_slot(4 * kg + j, r)] = rows4_sum(dBp[0], dBp[1], dBp[2], dBp[3]);
            if constexpr (kVC) wgC[wg_slot(4 * kg + j, r)] = rows4_sum(dCp[0], dCp[1], dCp[2], dCp[3]);
            if constexpr ((kg & 1) == 0) {           // half hh is written: read it back
                float2 (&tv)[8] = hh ? tv1 : tv0;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int n = 2 * i + tnh;
                    tv[i] = *reinterpret_cast<const float2*>(trh + n * 16 + 4 * (tm ^ (n >> 2)) + 2 * te);
                }
            }
        });
        gacar = ga;
        // keep the sums below after the whole adjoint, so the reads of the
        // first half have that time to land
        __builtin_amdgcn_sched_barrier(0);

        __builtin_amdgcn_s_setprio(0);
        // sums over states: lane r ends with step r of the chunk
        auto half_sum = [&](const float2 (&tv)[8], float& t1, float& t2) {
            const float a0 = tv[0].x + tv[4].x, a1 = tv[1].x + tv[5].x;
            const float a2_ = tv[2].x + tv[6].x, a3 = tv[3].x + tv[7].x;
            const float s1 = (a0 + a2_) + (a1 + a3);
            float e0 = Aw[0] * tv[0].y, e1 = Aw[1] * tv[1].y;
            e0 = __builtin_fmaf(Aw[2], tv[2].y, e0);
            e1 = __builtin_fmaf(Aw[3], tv[3].y, e1);
            e0 = __builtin_fmaf(Aw[4], tv[4].y, e0);
            e1 = __builtin_fmaf(Aw[5], tv[5].y, e1);
            e0 = __builtin_fmaf(Aw[6], tv[6].y, e0);
            e1 = __builtin_fmaf(Aw[7], tv[7].y, e1);
            const float s2 = e0 + e1;
            t1 = s1 + row_ror8(s1);
            t2 = s2 + row_ror8(s2);
        };
        float t1a, t2a, t1b, t2b;
        half_sum(tv1, t1a, t2a);
        half_sum(tv0, t1b, t2b);
        float s1r = tnh ? t1a : t1b;
        float s2r = tnh ? t2a : t2b;
        const bool in = !kTail || ck * kT + r < L;
        if constexpr (kAcc) {
            s1r += acc1;
            s2r += acc2v;
            if (in) {
                bstore<float>(Rao, oacc, uint32_t(ck * kT) * 4u, s1r);
                bstore<float>(Rao, oacc, uint32_t(ck * kT) * 4u + acc2, s2r);
            }
        }

        // ---- per-step outputs of step 16 ck + r
        const float du = Dv * dy + dt * s1r;
        const float ddt = uu * s1r + s2r;
        const float dd = softplus ? ddt * sigmoidf_(pre) : ddt;
        const uint32_t so = uint32_t(ck * kT) * es;
        if (in) {
            bstore<IT>(Rdu, odu, so, du);
            bstore<IT>(Rdd, odd, so, dd);
            if constexpr (kZ) bstore<IT>(Rdz, odz, so, dout * yv * sgz * (1.f + zz * (1.f - sgz)));
        }
        dD_acc += dy * uu;
        db_acc += in ? dd : 0.f;

        // B / C tile of the next chunk (ck - 1) into the other buffer
        stage(nxt, buf ^ 1);
    };

    // chunks k1 - 1, k1 - 2 first; two buffers of inputs alternate roles
    Chunk PA, PB;
    fetch_tail(k1 - 1, PA);
    fetch_tail(k1 - 2, PB);
    // the first flush (of the nonexistent chunk k1) adds these zeros to chunk k1 - 1
#pragma unroll
    for (int i = 0; i < 8; ++i) s_wg[i * kThreads + tid] = 0.f;     // buffer k1 & 1 = 0
    stage(PA, 1);
    // the first two pairs hold every output of the tail chunks (their dB / dC
    // are flushed one chunk later); k0, k1 even: ck odd, then even
    const int kt_end = k1 - 4 > k0 ? k1 - 4 : k0;
    int ck = k1 - 1;
    for (; ck > kt_end; ck -= 2) {
        chunk(ck, PA, PB, std::integral_constant<int, 1>{}, std::true_type{});
        chunk(ck - 1, PB, PA, std::integral_constant<int, 0>{}, std::true_type{});
    }
    for (; ck > k0; ck -= 2) {
        chunk(ck, PA, PB, std::integral_constant<int, 1>{}, std::false_type{});
        chunk(ck - 1, PB, PA, std::integral_constant<int, 0>{}, std::false_type{});
    }
    if constexpr (kVB || kVC) {
        lds_barrier();
        flush(k0, 0);
    }
    if constexpr (!kVB) atomicAdd(q.dB + c * kT + r, dBc);
    if constexpr (!kVC) atomicAdd(q.dC + c * kT + r, dCc);

    // ---- per-channel and per-(channel, state) sums over time and batch
    dD_acc = row_allsum(dD_acc);
    db_acc = row_allsum(db_acc);
    if constexpr (kDet) {
        // this (batch row, segment)'s partials: row b * nseg + seg of det_par
        float* pr = q.det_par + (b * nseg + seg) * p.dim * (kT + 2);
        pr[c * kT + r] = dA_acc;
        if (r == 0) {
            pr[p.dim * kT + c] = dD_acc;
            pr[p.dim * (kT + 1) + c] = db_acc;
        }
    } else {
        if (r == 0) {
            if (q.dD) atomicAdd(q.dD + c, dD_acc);
            if (q.ddelta_bias) atomicAdd(q.ddelta_bias + c, db_acc);
        }
        atomicAdd(q.dA + c * (kAcc ? q.dA_N : int64_t(kT)) + r, dA_acc);
    }
}

// Deterministic sums of the dA, dD, ddelta_bias partials: element i of
// [dA (dim * 16), dD (dim), ddelta_bias (dim)] is the sum of the rows'
// entries in row order, then added to the accumulator or, with overwrite,
// stored in its place.  dA rows are dA_N floats apart (16, or the call's
// dstate for a pass of a state-sliced backward, whose dA is based at its
// slice's first state).
__global__ __launch_bounds__(256) void ss_det_param_reduce(const float* __restrict__ par, int rows, int64_t dim,
                                                           float* __restrict__ dA, float* __restrict__ dD,
                                                           float* __restrict__ db, int overwrite, int64_t dA_N) {
    const int64_t n = dim * (kT + 2);
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
        float* dst = i < dim * kT ? dA + (i / kT) * dA_N + i % kT
                                  : (i < dim * (kT + 1) ? dD + (i - dim * kT) : db + (i - dim * (kT + 1)));
        if (i >= dim * kT && i < dim * (kT + 1) && !dD) continue;
        if (i >= dim * (kT + 1) && !db) continue;
        float s = 0.f;
        for (int k = 0; k < rows; ++k) s += par[int64_t(k) * n + i];
        *dst = overwrite ? s : *dst + s;
    }
}

// Pass A of the sequence-parallel backward: workgroup (b, seg, 16 channels)
// runs the adjoint recurrence over segment seg (segments 1 .. nseg - 1: the
// carry of the first segment leaves the sequence) from a zero carry, last
// step first, with the fast backward's lane layout and arithmetic but
// nothing else (no recomputed state, no gradients), and writes the carry it
// leaves at the segment's first step, g_t a_t, to seg_h and the segment's
// sum of delta' to seg_s.  kVC false: C constant ((dim, dstate) fp32, in a
// register; no tile, no barrier).
template <typename IT, bool kZ, bool kVC>
__global__ __launch_bounds__(kThreads, 3) void ss_bwd_seg_carry(const BwdParams q) {
    __shared__ __attribute__((aligned(16))) float s_c[2 * 16 * kT];                  // [buf][n][t]
    const FwdParams& p = q.f;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int r = lane & 15;
    const int j = lane >> 4;
    const int row = w * kRows + j;
    const int64_t nblk = p.dim / kChPerWG;
    const int nsa = p.nseg - 1;
    const int64_t blk = xcd_block_id();
    const int64_t bs = blk / nblk;
    const int64_t b = bs / nsa;
    const int seg = int(bs % nsa) + 1;
    const int64_t c0 = (blk % nblk) * kChPerWG;
    const int64_t c = c0 + row;
    const int64_t g = c0 / p.dpg;
    const int npairs = int((p.seqlen + 2 * kT - 1) / (2 * kT));   // chunk pairs, padded as in ss_bwd_fast
    const int k0 = 2 * seg_begin(seg, npairs, p.nseg), k1 = 2 * seg_begin(seg + 1, npairs, p.nseg);

    constexpr int64_t es64 = sizeof(IT);
    const rsrc_t Rd = make_rsrc_in(p.delta, (b * p.dl_bs + c0 * p.dl_ds) * es64, p.dl_end);
    const rsrc_t Ro = make_rsrc_in(q.dout, (b * q.do_bs + c0 * q.do_ds) * es64, q.do_end);
    const rsrc_t Rz = kZ ? make_rsrc_in(p.z, (b * p.z_bs + c0 * p.z_ds) * es64, p.z_end) : make_rsrc_n(nullptr, 0);
    const rsrc_t RC = kVC ? make_rsrc_in(p.C, (b * p.C_bs + g * p.C_gs) * es64, p.C_end) : make_rsrc_n(nullptr, 0);
    constexpr uint32_t es = sizeof(IT);

    const float bias = p.delta_bias ? p.delta_bias[c] : 0.f;
    const float a2 = p.A[c * p.A_ds + r * p.A_ns] * kLog2e;
    const bool softplus = p.softplus != 0;
    const float cconst = kVC ? 0.f : static_cast<const float*>(p.C)[c * p.C_gs + r * p.C_ns];

    struct Ck { float d, o, z, C; };
    // steps past a ragged sequence's end (the last segment's last chunks) are
    // identity steps: delta' = 0, dout = 0, C = 0, loads clamped to the end.
    // Chunks wholly inside the sequence load at a fixed per-lane offset plus
    // the chunk's uniform offset (no per-load address arithmetic).
    const int64_t L = p.seqlen;
    const uint32_t od = uint32_t(row * p.dl_ds + r) * es, oo = uint32_t(row * q.do_ds + r) * es;
    const uint32_t oz = uint32_t(row * p.z_ds + r) * es, oC = uint32_t(row * p.C_ns + r) * es;
    auto fetch = [&](int ck, Ck& P) {
        if (int64_t(ck) * kT + kT <= L) {
            const uint32_t so = uint32_t(ck * kT) * es;
            P.d = bload<IT>(Rd, od, so);
            P.o = bload<IT>(Ro, oo, so);
            P.z = kZ ? bload<IT>(Rz, oz, so) : 0.f;
            P.C = kVC ? bload<IT>(RC, oC, so) : 0.f;
            return;
        }
        const int t = ck * kT + r;
        const bool in = t < L;
        const int te = in ? t : int(L) - 1;
        P.d = in ? bload<IT>(Rd, uint32_t(row * p.dl_ds + te) * es, 0) : (softplus ? -INFINITY : -bias);
        P.o = in ? bload<IT>(Ro, uint32_t(row * q.do_ds + te) * es, 0) : 0.f;
        P.z = kZ && in ? bload<IT>(Rz, uint32_t(row * p.z_ds + te) * es, 0) : 0.f;
        P.C = (kVC && in) ? bload<IT>(RC, uint32_t(row * p.C_ns + te) * es, 0) : 0.f;
    };
    auto stage = [&](const Ck& P, int buf) {
        if constexpr (kVC) s_c[buf * 16 * kT + bc_slot(row, r)] = P.C;
    };

    float ga = 0.f, dsum = 0.f;
    Ck P;
    fetch(k1 - 1, P);
    stage(P, 0);
    for (int ck = k1 - 1; ck >= k0; --ck) {
        const int buf = (k1 - 1 - ck) & 1;
        if constexpr (kVC) lds_barrier();   // C tile of ck staged
        const Ck cur = P;
        fetch(ck > k0 ? ck - 1 : k0, P);
        float Cq[kT];
        const float* sC = s_c + buf * 16 * kT;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (kVC) {
                const float4 vc = *reinterpret_cast<const float4*>(sC + bc_slot(r, 4 * i));
                Cq[4 * i] = vc.x; Cq[4 * i + 1] = vc.y; Cq[4 * i + 2] = vc.z; Cq[4 * i + 3] = vc.w;
            } else {
                // (past a ragged end the steps are identity steps with dout 0)
                Cq[4 * i] = Cq[4 * i + 1] = Cq[4 * i + 2] = Cq[4 * i + 3] = cconst;
            }
        }
        const float pre = cur.d + bias;
        float dt = softplus ? softplus20(pre) : pre;
        float dy = kZ ? cur.o * cur.z * sigmoidf_(cur.z) : cur.o;
        dsum += dt;
        dpp_sources_ready(dt, dy, dsum);
        // the carry's chain at raised wave priority (as in the full backward;
        // 1 x 1536 x 32768 bf16 backward with segments 862 -> 834 us)
        __builtin_amdgcn_s_setprio(1);
        float as[kT];
        static_for<kT>([&](auto K) {
            constexpr int k = decltype(K)::value;
            as[k] = __builtin_amdgcn_exp2f(row_bcast<k>(dt) * a2);
        });
        static_for<kT>([&](auto K) {
            constexpr int k = kT - 1 - decltype(K)::value;
            float gv = ga;
            bfmac<k>(gv, dy, Cq[k]);             // g_t = a_{t+1} g_{t+1} + dy_t C_t
            ga = gv * as[k];
        });
        __builtin_amdgcn_s_setprio(0);
        stage(P, buf ^ 1);
    }
    const int64_t si = (b * p.nseg + seg) * p.dim + c;
    p.seg_h[si * kT + r] = ga;
    dsum = row_allsum(dsum);                       // the row's 16 lanes hold one step each
    if (r == 0) p.seg_s[si] = dsum;
}

bool bwd_fast_ok(const BwdParams& q);

// Segments for the backward (seg_count): whole chunk pairs, at least 8
// pairs (16 chunks) each.
int bwd_segments(const BwdParams& q) {
    if (!bwd_fast_ok(q)) return 1;
    const FwdParams& p = q.f;
    return seg_count(p.batch * (p.dim / kChPerWG), (p.seqlen + 2 * kT - 1) / (2 * kT), 8);
}

bool bwd_fast_ok(const BwdParams& q) {
    const FwdParams& p = q.f;
    // every byte offset the kernel forms stays below 2^32: rows and seqlen
    // below 2^26 elements, checkpoints addressed from their own chunk (dim
    // below 2^24)
    // (a seqlen that is not a multiple of 32 ends in identity-padded chunks)
    // (deterministic sums only with B and C both variable)
    return p.dstate == 16 && ((p.var_B && p.var_C) || !q.det) && p.seqlen >= 1 &&
           p.dim % kChPerWG == 0 && p.dpg % kChPerWG == 0 && (!p.has_z || p.y != nullptr) &&
           small_strides({p.seqlen + 2 * kT, p.u_ds, p.dl_ds, p.z_ds, p.y_ds, p.B_ns, p.C_ns,
                          q.do_ds, q.du_ds, q.dd_ds, q.dz_ds}) &&
           p.dim * p.xN < (int64_t(1) << 28);
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
// each), the slices summed in order first; `overwrite` ignores what dB / dC
// held.
__global__ __launch_bounds__(256) void ss_ws_reduce(const float4* __restrict__ ws, int slices, int64_t n4,
                                                    float4* __restrict__ dB, float4* __restrict__ dC,
                                                    int overwrite) {
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
        float4 sb = ws[i], sc = ws[n4 + i];
        for (int k = 1; k < slices; ++k) {
            const float4 vb = ws[(2 * k) * n4 + i], vc = ws[(2 * k + 1) * n4 + i];
            sb.x += vb.x; sb.y += vb.y; sb.z += vb.z; sb.w += vb.w;
            sc.x += vc.x; sc.y += vc.y; sc.z += vc.z; sc.w += vc.w;
        }
        if (!overwrite) {
            const float4 ob = dB[i], oc = dC[i];
            sb.x += ob.x; sb.y += ob.y; sb.z += ob.z; sb.w += ob.w;
            sc.x += oc.x; sc.y += oc.y; sc.z += oc.z; sc.w += oc.w;
        }
        dB[i] = sb;
        dC[i] = sc;
    }
}

// As ss_ws_reduce for slices whose rows are padded to ld floats (or dB / dC
// not 16-byte aligned): element t < seqlen of row i of the slices (16 state
// rows per batch row and group) is the sum of the slices' element i * ld + t,
// in slice order, then added to what dB / dC held unless overwrite, at row
// (i / 16) * N + i % 16 of dB / dC (N state rows per batch row and group; a
// pass of a state-sliced backward passes dB / dC based at its slice's first
// state).  A workgroup per row.
__global__ __launch_bounds__(256) void ss_ws_reduce_rows(const float* __restrict__ ws, int slices, int64_t stride,
                                                         int64_t rows, int64_t L, int64_t ld, float* __restrict__ dB,
                                                         float* __restrict__ dC, int overwrite, int64_t N) {
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const int64_t orow = (row / kT) * N + row % kT;
        for (int64_t t = threadIdx.x; t < L; t += blockDim.x) {
            const int64_t w = row * ld + t, o = orow * L + t;
            float sb = ws[w], sc = ws[stride + w];
            for (int k = 1; k < slices; ++k) {
                sb += ws[2 * k * stride + w];
                sc += ws[(2 * k + 1) * stride + w];
            }
            if (!overwrite) {
                sb += dB[o];
                sc += dC[o];
            }
            dB[o] = sb;
            dC[o] = sc;
        }
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
    // deterministic sums: every slice element is written, and the fixed-order
    // passes overwrite (zero_grads) or add to the accumulators themselves
    if (sliced && !p.det) add(p.ws, 2 * p.ws_slices * p.ws_stride);
    if (p.zero_grads && !p.det) {
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
    if (!bwd_fast_ok(p) || !p.f.var_B || !p.f.var_C) return 1;   // (slices only with B and C both variable)
    if (p.det) return int(p.f.dpg / kChPerWG);   // one slice per channel block of a group
    // at most 96 channel blocks per slice: each workgroup adds once per
    // (state, step) and chunk, so the contention of up to 96 adders per
    // address costs less than clearing and summing more slices (measured on
    // MI355X, same process: dim 1536 fp32 backward 405 us with 8 slices,
    // 397 us with one; dim 5120 bf16 2462 us with 16, 2441 us with 4)
    const int64_t blocks = p.f.dpg / kChPerWG;
    const int64_t k = (blocks + 95) / 96;
    return int(k < 1 ? 1 : (k > 16 ? 16 : k));
}

// the fast backward for the combination of variable / constant B and C
template <typename IT, bool kZ>
static void launch_bwd_bc(const BwdParams& p, dim3 grid, dim3 block, hipStream_t stream) {
    const FwdParams& f = p.f;
    if (f.var_B && f.var_C) hipLaunchKernelGGL((ss_bwd_fast<IT, kZ, false, false, true, true>), grid, block, 0, stream, p);
    else if (f.var_B) hipLaunchKernelGGL((ss_bwd_fast<IT, kZ, false, false, true, false>), grid, block, 0, stream, p);
    else if (f.var_C) hipLaunchKernelGGL((ss_bwd_fast<IT, kZ, false, false, false, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((ss_bwd_fast<IT, kZ, false, false, false, false>), grid, block, 0, stream, p);
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
        // the slice sum as whole float4 rows: rows of seqlen floats, 16-byte
        // aligned dB / dC
        const bool flat = p.bc_ld == p.f.seqlen && p.f.xN == kT && (reinterpret_cast<uintptr_t>(p.dB) & 15) == 0 &&
                          (reinterpret_cast<uintptr_t>(p.dC) & 15) == 0;
        const int64_t n4 = sliced && flat ? p.ws_stride / 4 : 0;
        const unsigned rgrid = unsigned(n4 > 0 ? (n4 + 255) / 256 < 2048 ? (n4 + 255) / 256 : 2048 : 1);
        const int nseg = p.f.nseg > 1 ? p.f.nseg : 1;
        if (nseg > 1) {
            const dim3 agrid(unsigned(nblk * p.f.batch * (nseg - 1)));
            if (p.f.var_C) {
                if (p.f.has_z) hipLaunchKernelGGL((ss_bwd_seg_carry<IT, true, true>), agrid, block, 0, stream, p);
                else hipLaunchKernelGGL((ss_bwd_seg_carry<IT, false, true>), agrid, block, 0, stream, p);
            } else {
                if (p.f.has_z) hipLaunchKernelGGL((ss_bwd_seg_carry<IT, true, false>), agrid, block, 0, stream, p);
                else hipLaunchKernelGGL((ss_bwd_seg_carry<IT, false, false>), agrid, block, 0, stream, p);
            }
        }
        const dim3 sgrid(unsigned(nblk * p.f.batch * nseg));
        if (p.det && p.f.acc) {
            if (p.f.has_z) hipLaunchKernelGGL((ss_bwd_fast<IT, true, true, true, true, true>), sgrid, block, 0, stream, p);
            else hipLaunchKernelGGL((ss_bwd_fast<IT, false, true, true, true, true>), sgrid, block, 0, stream, p);
        } else if (p.det) {
            if (p.f.has_z) hipLaunchKernelGGL((ss_bwd_fast<IT, true, true, false, true, true>), sgrid, block, 0, stream, p);
            else hipLaunchKernelGGL((ss_bwd_fast<IT, false, true, false, true, true>), sgrid, block, 0, stream, p);
        } else if (p.f.acc) {
            if (p.f.has_z) hipLaunchKernelGGL((ss_bwd_fast<IT, true, false, true, true, true>), sgrid, block, 0, stream, p);
            else hipLaunchKernelGGL((ss_bwd_fast<IT, false, false, true, true, true>), sgrid, block, 0, stream, p);
        } else if (p.f.has_z) {
            launch_bwd_bc<IT, true>(p, sgrid, block, stream);
        } else {
            launch_bwd_bc<IT, false>(p, sgrid, block, stream);
        }
        if (p.det) {
            const int64_t n = p.f.dim * (kT + 2);
            const unsigned pgrid = unsigned((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024);
            hipLaunchKernelGGL(ss_det_param_reduce, dim3(pgrid), dim3(256), 0, stream, p.det_par,
                               int(p.f.batch * nseg), p.f.dim, p.dA, p.dD, p.ddelta_bias, int(p.zero_grads),
                               p.f.acc ? p.dA_N : int64_t(kT));
        }
        if (sliced && flat) {
            hipLaunchKernelGGL(ss_ws_reduce, dim3(rgrid), dim3(256), 0, stream,
                               reinterpret_cast<const float4*>(p.ws), int(p.ws_slices), n4,
                               reinterpret_cast<float4*>(p.dB), reinterpret_cast<float4*>(p.dC),
                               int(p.zero_grads));
        } else if (sliced) {
            const int64_t rows = p.f.batch * (p.f.dim / p.f.dpg) * kT;
            hipLaunchKernelGGL(ss_ws_reduce_rows, dim3(unsigned(rows < 2048 ? rows : 2048)), dim3(256), 0, stream,
                               p.ws, int(p.ws_slices), p.ws_stride, rows, p.f.seqlen, p.bc_ld, p.dB, p.dC,
                               int(p.zero_grads), p.f.xN);
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
