// Forward selective scan for gfx950.
//
// Semantics follow the reference forward kernel
// (csrc/selective_scan/forward_kernel.cu:174-310) plus the z gate applied by
// its caller (modules/mamba_simple.py:143-146):
//   delta' = softplus(delta + bias), a = exp2(delta' * A * log2 e),
//   h_t = a_t h_{t-1} + delta'_t u_t B_t,  y_t = sum_n C_t h_t + D u_t,
//   out = y * silu(z).
//
// Work decomposition (not the reference's one-block-per-(b, d) CUB scan): a
// lane owns one (channel, state) recurrence and walks time sequentially, so
// there is no cross-lane scan at all.  A 16-lane row is one channel; per
// 16-step tile, lane r loads the per-step inputs of step t0 + r and the
// other lanes read them with DPP row broadcasts folded into the arithmetic.
// The sum over states, y_t = sum_n C h, is an in-row transposed sum through
// LDS.  Every kChunk steps the state is checkpointed to x for the backward;
// with a z gate the pre-gate output y is also saved for the backward's dz.
#include "ss_device.hpp"
#include "ss_kernels.hpp"

namespace ss {

// kVarBC: B and C are both variable (the common case, no runtime switches).
template <typename IT, int SPL, bool kVarBC>
__global__ __launch_bounds__(kThreads) void ss_fwd_kernel(const FwdParams p) {
    __shared__ __attribute__((aligned(16))) float tr_buf[kWaves * 2 * kTrWave];

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
    float* wbuf = tr_buf + w * 2 * kTrWave;

    const IT* u = static_cast<const IT*>(p.u) + b * p.u_bs + c * p.u_ds;
    const IT* dl = static_cast<const IT*>(p.delta) + b * p.dl_bs + c * p.dl_ds;
    // without a z gate zp aliases u so that its (unused) load stays unconditional
    const IT* zp = p.has_z ? static_cast<const IT*>(p.z) + b * p.z_bs + c * p.z_ds : u;
    IT* out = static_cast<IT*>(p.out) + b * p.o_bs + c * p.o_ds;
    IT* ysave = (p.has_z && p.y) ? static_cast<IT*>(p.y) + b * p.y_bs + c * p.y_ds : nullptr;
    const IT* Bv_base = static_cast<const IT*>(p.B) + b * p.B_bs + g * p.B_gs;
    const IT* Cv_base = static_cast<const IT*>(p.C) + b * p.C_bs + g * p.C_gs;
    const float* Bc_base = static_cast<const float*>(p.B) + c * p.B_gs;  // constant B: (dim, dstate)
    const float* Cc_base = static_cast<const float*>(p.C) + c * p.C_gs;
    // x: (batch, chunk, dim, dstate); not written when null
    float* xrow = p.x ? p.x + (b * p.n_chunks * p.dim + c) * N : nullptr;
    const int64_t x_chunk_stride = p.dim * N;

    const float Dv = p.D ? p.D[c] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[c] : 0.f;

    float A2[SPL], Bc[SPL], Cc[SPL], h[SPL];
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
        const int n = 16 * s + r;
        const bool nv = n < N;
        A2[s] = nv ? p.A[c * p.A_ds + n * p.A_ns] * kLog2e : 0.f;
        Bc[s] = (!p.var_B && nv) ? Bc_base[n * p.B_ns] : 0.f;
        Cc[s] = (!p.var_C && nv) ? Cc_base[n * p.C_ns] : 0.f;
        h[s] = 0.f;
    }

    // Inputs of one 16-step tile: the per-step values of step t0 + r owned by
    // this lane, and (single state group) the B / C rows of this lane's state.
    struct Tile {
        float u, dl, z;
        float B[kT], C[kT];
    };
    // Padding states (n >= dstate: the last group's lanes past dstate % 16,
    // or a whole group when dstate is below 16 SPL, e.g. 48 on SPL 4) read a
    // valid row and get C = 0, so their h never reaches y or x.
    const bool pad_states = N < 16 * SPL;
    auto load_bc = [&](int64_t t0, int s, float (&Bo)[kT], float (&Co)[kT]) {
        const int n = 16 * s + r;
        const bool nv = n < N;
        const int nn = nv ? n : N - 1;
        if (kVarBC || p.var_B) load_tile16<IT>(Bv_base + nn * p.B_ns, t0, L, p.vec_B != 0, Bo);
        else {
#pragma unroll
            for (int k = 0; k < kT; ++k) Bo[k] = Bc[s];
        }
        if (kVarBC || p.var_C) load_tile16<IT>(Cv_base + nn * p.C_ns, t0, L, p.vec_C != 0, Co);
        else {
#pragma unroll
            for (int k = 0; k < kT; ++k) Co[k] = Cc[s];
        }
        if (pad_states && !nv) {
#pragma unroll
            for (int k = 0; k < kT; ++k) Co[k] = 0.f;
        }
    };
    // Loads are unconditional (addresses clamped inside the sequence past its
    // end), so prefetches beyond the last tile are harmless.
    auto load_tile = [&](int64_t t0, Tile& T) {
        const int64_t t = t0 + r;
        if (t0 + kT <= L) {
            T.u = load_at(u, t);
            T.dl = load_at(dl, t);
            T.z = load_at(zp, t);
        } else {
            T.u = load_or0(u, t, L);
            T.dl = load_or0(dl, t, L);
            T.z = load_or0(zp, t, L);
        }
        if constexpr (SPL == 1) load_bc(t0, 0, T.B, T.C);
    };
    // The sum over states of a tile is written to LDS at the end of the tile
    // and read back in the middle of the next one, so its latency overlaps
    // that tile's arithmetic; two scratch slots alternate.  (The slot is
    // applied as an offset to the __shared__ array itself: a pointer picked
    // from an array of pointers would lose its LDS address space and turn
    // into slow flat loads.)
    int64_t pend_t = -1;          // step of the pending output (this lane), -1 if none
    float pend_u = 0.f, pend_z = 0.f;
    auto finish_pending = [&](int slot) {
        if (pend_t < 0) return;
        const float y = row_transpose_read(wbuf + slot * kTrWave, j, r);
        if (pend_t < L && cval) {
            float o = y + Dv * pend_u;
            if (p.has_z) {
                if (ysave) io<IT>::store(ysave + pend_t, o);
                o *= pend_z * sigmoidf_(pend_z);
            }
            io<IT>::store(out + pend_t, o);
        }
    };

    auto compute_tile = [&](int64_t t0, Tile& T, int slot) {
        float dt = T.dl + bias;
        if (p.softplus) dt = softplus20(dt);
        if (t0 + r >= L) dt = 0.f;               // identity step: a = 1, b = 0
        const float dtu = dt * T.u;

        float yp[kT];
#pragma unroll
        for (int k = 0; k < kT; ++k) yp[k] = 0.f;
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
            const int n = 16 * s + r;
            float Bl[kT], Cl[kT];
            if constexpr (SPL > 1) load_bc(t0, s, Bl, Cl);
            const float (&Bt)[kT] = (SPL == 1) ? T.B : Bl;
            const float (&Ct)[kT] = (SPL == 1) ? T.C : Cl;
            const float a2 = A2[s];
            // decay factors and inputs of all 16 steps first: they do not
            // depend on h, so the exp latency is off the h chain
            float a[kT], bb[kT];
            static_for<kT>([&](auto K) {
                constexpr int k = decltype(K)::value;
                a[k] = __builtin_amdgcn_exp2f(row_bcast<k>(dt) * a2);
                bb[k] = row_bcast<k>(dtu) * Bt[k];
            });
            if (s == 0) finish_pending(slot ^ 1);
            float hs = h[s];
            static_for<kT>([&](auto K) {
                constexpr int k = decltype(K)::value;
                hs = __builtin_fmaf(a[k], hs, bb[k]);
                yp[k] = __builtin_fmaf(Ct[k], hs, yp[k]);
            });
            h[s] = hs;
            const bool chunk_end = ((t0 + kT) % kChunk == 0) || (t0 + kT >= L);
            if (chunk_end && cval && n < N && p.x) xrow[(t0 / kChunk) * x_chunk_stride + n] = hs;
            if (t0 + kT >= L && cval && n < N && p.last_state) p.last_state[(b * p.dim + c) * N + n] = hs;
        }
        row_transpose_write(wbuf + slot * kTrWave, yp, j, r);
        pend_t = t0 + r;
        pend_u = T.u;
        pend_z = T.z;
    };

    // two tile buffers, alternated by unrolling the time loop twice: the
    // loads of a tile are issued one tile before it is computed
    Tile T0, T1;
    load_tile(0, T0);
    int slot = 0;
    for (int64_t t0 = 0; t0 < L; t0 += 2 * kT) {
        load_tile(t0 + kT, T1);
        compute_tile(t0, T0, slot);
        slot ^= 1;
        load_tile(t0 + 2 * kT, T0);
        if (t0 + kT < L) { compute_tile(t0 + kT, T1, slot); slot ^= 1; }
    }
    finish_pending(slot ^ 1);
}

// Fast path: dstate 16, variable B and C, dim and channels per group
// multiples of 16, z gate fixed at compile time.  Every step, state and
// channel of the main loop is real, so it has no branch around a memory
// access (on gfx950 the compiler waits for every outstanding load at such a
// branch, which would serialise the prefetch).  A seqlen that is not a
// multiple of 64 ends in a partial super-chunk, the tail, run once after the
// loop: its loads are clamped to the sequence and zero past it, its steps
// past the sequence are identity steps (decay 1, input 0, as the reference
// pads its last chunk: forward_kernel.cu:267-271), and its stores stop at
// the sequence's end.  The vector accesses need only element alignment:
// the HSA runtime runs the shader memory pipeline in its unaligned mode (the
// compiler itself emits 16-byte loads at byte-aligned addresses for this
// target), so rows at any element offset (an odd seqlen, a sliced view) keep
// the one-access-per-4-steps streams.
//
// Global traffic moves in 64-step super-chunks with one barrier each: lane r
// of a row owns steps 4r..4r+3 of its channel and reads / writes them as one
// 16-byte (fp32) access, so every row segment is 256 contiguous bytes (HBM
// streams of 64-byte segments reach only about 70 % of the bandwidth of
// 256-byte ones on this part).  Within a super-chunk, four 16-step chunks:
//  - step k of chunk q is owned by lane 4q + k/4, component k % 4, and
//    reaches the other lanes of the row by a DPP row broadcast of that lane;
//  - the B / C tile of the super-chunk is staged through LDS (double
//    buffered, loaded one super-chunk ahead);
//  - y_t = sum_n C h is an in-row transposition through LDS: each lane
//    writes its 16 states h_t, and lane r forms sum_n C h for step r one
//    chunk later (after the next chunk's decay factors, so the LDS round
//    trip is off the critical path), with C from a transposed copy of the
//    C tile; the lanes of the recurrence never touch C.  The 64 sums of a
//    super-chunk are regrouped through LDS into the owners' float4 for the
//    stores, one super-chunk late;
//  - the checkpoint of the state is one store per lane and chunk (a wave's
//    4 channels x 16 states are 256 contiguous bytes);
//  - out, y and the checkpoints are stored non-temporal: nothing in the
//    kernel reads them again (fp32 forward 145.5-150.2 -> 142.5-149.3 us,
//    bf16 933 -> 916 us, same box; the backward's stores measured no faster
//    that way and keep the default policy).
constexpr int kSC = 64;                      // steps per super-chunk
constexpr int kQ = kSC / kT;                 // chunks per super-chunk
constexpr int kYRow = kT * kT + 16;          // per-row product tile, padded so rows j, j + 1 use different bank halves
constexpr int kYoRow = kSC + 16;             // per-row regroup area, padded likewise

// LDS bank model of gfx950 (measured): 4-byte accesses see 32 banks of 4
// bytes, 8- and 16-byte accesses see 64.
// B / C super-chunk tile slot of (state n, 4-step group gi): the 16 lanes of
// states 0..15 reading group gi with ds_read_b128 cover all 64 banks once,
// and a staging row writing its 16 groups does too.
__device__ __forceinline__ int bc64_slot(int n, int gi) { return n * kSC + 4 * (gi ^ n); }
// Transposed C tile, [64 steps][16 states]: float4 i of step t (states
// 4i..4i+3) at t * 16 + 4 * (i ^ ((t >> 2) & 3)), so the 16 lanes of a row
// reading steps 16q..16q+15 with ds_read_b128 cover all 64 banks once.
__device__ __forceinline__ int ct_slot4(int t, int i) { return t * 16 + 4 * (i ^ ((t >> 2) & 3)); }

// kAcc: one pass of a state-sliced scan (dstate 16 S, one pass per 16-state
// slice): y is added to the sums over the earlier slices (p.acc, fp32) and,
// but in the last pass, stored back there instead of becoming out / y (whose
// extents the host sets to 0 then; D is applied in the last pass only).
// kVB / kVC: B / C vary per step (staged per super-chunk through LDS);
// false: constant, (dim, dstate) fp32, held in registers for the whole
// launch (each lane its channel's B of its state; the 16 C of its channel).
// With both constant the kernel has no B / C tile and no barrier.
// 16-bit I/O (not state-sliced): the B tile is read just before the state
// recurrence instead of ahead of the decay factors, which fits 128 VGPRs and
// so 4 workgroups per CU (bf16 forward about 5 % faster at 1,280 and 1,536
// workgroups; fp32, whose wider streams gain nothing from the fourth
// workgroup, keeps the early reads and 3 per CU).
template <typename IT, bool kAcc>
constexpr bool fwd_late_b() { return sizeof(IT) != 4 && !kAcc; }
template <typename IT, bool kZ, bool kAcc, bool kVB, bool kVC>
__global__ __launch_bounds__(kThreads, (fwd_late_b<IT, kAcc>() ? 4 : 3)) void ss_fwd_fast(const FwdParams p) {
    __shared__ __attribute__((aligned(16))) float s_bc[2 * 2 * 16 * kSC];          // [buf][B [n][64 steps], C [64 steps][n]]
    __shared__ __attribute__((aligned(16))) float s_yp[kWaves * kRows * kYRow];    // [wave][row][n][16 steps]
    __shared__ __attribute__((aligned(16))) float s_yo[kWaves * kRows * kYoRow];   // [wave][row][64 steps]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int r = lane & 15;
    const int j = lane >> 4;
    const int row = w * kRows + j;                 // this lane's channel row in the workgroup
    const int64_t nblk = p.dim / kChPerWG;
    // logical workgroup (b, seg, channel block), channel block fastest: the
    // workgroups of one segment of one batch row read the same B / C
    const int64_t blk = xcd_block_id();
    const int nseg = p.nseg;
    const int64_t bs = blk / nblk;
    const int64_t b = bs / nseg;
    const int seg = int(bs % nseg);
    const int64_t c0 = (blk % nblk) * kChPerWG;
    const int64_t c = c0 + row;
    const int64_t g = c0 / p.dpg;
    // super-chunks, the last one partial when seqlen is not a multiple of 64
    // (below 2^20); the last segment ends with that partial one, the tail
    const int nsc_pad = int((p.seqlen + kSC - 1) / kSC);
    const int sc0 = seg_begin(seg, nsc_pad, nseg), sc1 = seg_begin(seg + 1, nsc_pad, nseg);
    const int lt = int(p.seqlen - int64_t(nsc_pad - 1) * kSC);   // steps of the last super-chunk, 1..64
    const bool tail = seg == nseg - 1 && lt < kSC;
    const int scf = tail ? sc1 - 1 : sc1;                       // end of the full super-chunks

    // buffer resources at the workgroup's rows; lane (row, r) owns steps
    // 4r..4r+3 of channel c0 + row and, for the B / C staging, of state row
    constexpr int64_t es64 = sizeof(IT);
    const rsrc_t Ru = make_rsrc_in(p.u, (b * p.u_bs + c0 * p.u_ds) * es64, p.u_end);
    const rsrc_t Rd = make_rsrc_in(p.delta, (b * p.dl_bs + c0 * p.dl_ds) * es64, p.dl_end);
    const rsrc_t Rz = kZ ? make_rsrc_in(p.z, (b * p.z_bs + c0 * p.z_ds) * es64, p.z_end) : make_rsrc_n(nullptr, 0);
    const rsrc_t RB = kVB ? make_rsrc_in(p.B, (b * p.B_bs + g * p.B_gs) * es64, p.B_end) : make_rsrc_n(nullptr, 0);
    const rsrc_t RC = kVC ? make_rsrc_in(p.C, (b * p.C_bs + g * p.C_gs) * es64, p.C_end) : make_rsrc_n(nullptr, 0);
    // out / y are written with 16-byte stores, which take their advance in the
    // resource base and no uniform offset (see bstore4).  Without a y (or x)
    // buffer the stores go through a zero-byte resource and are dropped: a
    // forward that no backward follows writes neither.
    const int64_t o_off = (b * p.o_bs + c0 * p.o_ds) * es64, y_off = (b * p.y_bs + c0 * p.y_ds) * es64;
    const int64_t y_end = kZ ? p.y_end : 0;
    // x: (batch, chunk, dim, xN), this pass's 16 states at p.x (xN is 16
    // unless the call is state-sliced)
    const int64_t xN = kAcc ? p.xN : kT;
    const int64_t x_off = (b * p.n_chunks * p.dim + c0) * xN * 4;
    constexpr uint32_t es = sizeof(IT);
    const uint32_t ou = uint32_t(row * p.u_ds + 4 * r) * es, od = uint32_t(row * p.dl_ds + 4 * r) * es;
    const uint32_t oz = uint32_t(row * p.z_ds + 4 * r) * es;
    const uint32_t oB = uint32_t(row * p.B_ns + 4 * r) * es, oC = uint32_t(row * p.C_ns + 4 * r) * es;
    const uint32_t oo = uint32_t(row * p.o_ds + 4 * r) * es, oy = uint32_t(row * p.y_ds + 4 * r) * es;
    const uint32_t ox = uint32_t(row * xN + r) * 4u;
    const int64_t x_chunk_bytes = p.dim * xN * 4;          // below 2^34 (dim below 2^24, xN at most 256)
    // the tail's checkpoints: a resource that ends with this batch row's
    // n_chunks chunks, so the stores of chunks past the sequence are dropped
    const int64_t x_row_end = ((b + 1) * p.n_chunks * p.dim * xN - (xN - kT)) * 4;
    const int64_t x_tail_end = p.x_end < x_row_end ? p.x_end : x_row_end;
    // the checkpoints through resources based at a window of super-chunks
    // whose offsets stay below p.x_win (2^31 bytes unless the caller set a
    // smaller span; offsets from the row's first chunk would pass 2^32 once
    // seqlen x dim reaches 2^30); a window is rebased when a super-chunk
    // leaves it, which at most rows never happens
    const int x_wsc = int(p.x_win / (kQ * x_chunk_bytes)) > 0 ? int(p.x_win / (kQ * x_chunk_bytes)) : 1;
    int x_w0 = sc0;
    rsrc_t Rx_w = make_rsrc_in(p.x, x_off + int64_t(kQ * sc0) * x_chunk_bytes, p.x_end);
    rsrc_t Rx_wt = make_rsrc_in(p.x, x_off + int64_t(kQ * sc0) * x_chunk_bytes, x_tail_end);

    const float Dv = p.D ? p.D[c] : 0.f;
    const float bias = p.delta_bias ? p.delta_bias[c] : 0.f;
    const float a2 = p.A[c * p.A_ds + r * p.A_ns] * kLog2e;
    const bool softplus = p.softplus != 0;
    // constant B: this lane's B[c][r]
    const float bconst = kVB ? 0.f : static_cast<const float*>(p.B)[c * p.B_gs + r * p.B_ns];

    struct Super { float4 u, d, z, B, C; };
    auto fetch = [&](int sc, Super& S) {       // 0 <= sc < nsc
        const uint32_t so = uint32_t(sc * kSC) * es;
        S.u = bload4<IT>(Ru, ou, so);
        S.d = bload4<IT>(Rd, od, so);
        S.z = kZ ? bload4<IT>(Rz, oz, so) : make_float4(0.f, 0.f, 0.f, 0.f);
        S.B = kVB ? bload4<IT>(RB, oB, so) : make_float4(0.f, 0.f, 0.f, 0.f);
        S.C = kVC ? bload4<IT>(RC, oC, so) : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    // the tail super-chunk sc: element loads at offsets clamped to its lt
    // steps, zero past them
    auto fetch_tail = [&](int sc, Super& S) {
        const uint32_t so = uint32_t(sc * kSC) * es;
        float v[5][4];
        const int64_t rs[5] = {row * p.u_ds, row * p.dl_ds, row * p.z_ds, row * p.B_ns, row * p.C_ns};
        const rsrc_t R[5] = {Ru, Rd, Rz, RB, RC};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = 4 * r + i;
            const int tc = t < lt ? t : lt - 1;
#pragma unroll
            for (int k = 0; k < 5; ++k) {
                const float x = ((k == 2 && !kZ) || (k == 3 && !kVB) || (k == 4 && !kVC)) ? 0.f
                                                                       : bload<IT>(R[k], uint32_t(rs[k] + tc) * es, so);
                v[k][i] = t < lt ? x : 0.f;
            }
        }
        S.u = make_float4(v[0][0], v[0][1], v[0][2], v[0][3]);
        S.d = make_float4(v[1][0], v[1][1], v[1][2], v[1][3]);
        S.z = make_float4(v[2][0], v[2][1], v[2][2], v[2][3]);
        S.B = make_float4(v[3][0], v[3][1], v[3][2], v[3][3]);
        S.C = make_float4(v[4][0], v[4][1], v[4][2], v[4][3]);
    };
    auto stage = [&](const Super& S, int buf) {
        if constexpr (kVB) *reinterpret_cast<float4*>(s_bc + (buf * 2 + 0) * 16 * kSC + bc64_slot(row, r)) = S.B;
        if constexpr (kVC) {
            // C transposed: step 4r + i, state row
            float* ct = s_bc + (buf * 2 + 1) * 16 * kSC;
            const int ci = 4 * ((row >> 2) ^ (r & 3)) + (row & 3);
            ct[(4 * r + 0) * 16 + ci] = S.C.x;
            ct[(4 * r + 1) * 16 + ci] = S.C.y;
            ct[(4 * r + 2) * 16 + ci] = S.C.z;
            ct[(4 * r + 3) * 16 + ci] = S.C.w;
        }
    };
    // this row's product tile: lane n writes its steps 4m..4m+3 as a float4
    // at n * 16 + 4 * (m ^ ((n >> 1) & 3)); lane r reads step r of state n at
    // n * 16 + 4 * ((r >> 2) ^ ((n >> 1) & 3)) + (r & 3)
    float* yrow = s_yp + (w * kRows + j) * kYRow;
    float* yo = s_yo + (w * kRows + j) * kYoRow;
    int yoff[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) yoff[m] = 4 * ((r >> 2) ^ m) + (r & 3);

    // the state entering this segment: the earlier segments' end states
    // (each scanned from zero) joined in order, h <- exp(A sum delta') h + h_end
    float h = 0.f;
    for (int s2 = 0; s2 < seg; ++s2) {
        const int64_t si = (b * nseg + s2) * p.dim + c;
        h = __builtin_fmaf(__builtin_amdgcn_exp2f(a2 * p.seg_s[si]), h, p.seg_h[si * kT + r]);
    }
    float4 pu = make_float4(0.f, 0.f, 0.f, 0.f), pz = pu;   // u, z of the previous super-chunk

    // state slices (kAcc): this row's sums over the earlier slices, fp32
    // (batch, dim, seqlen) at p.acc; lane r's steps 4r..4r+3 of a super-chunk
    // are loaded right after the previous super-chunk's outputs, a
    // super-chunk ahead of their own
    const int64_t acc_off = (b * p.dim + c0) * p.seqlen * 4;
    const uint32_t oacc = uint32_t(row * p.seqlen + 4 * r) * 4u;
    float4 pacc = make_float4(0.f, 0.f, 0.f, 0.f);
    auto acc_load = [&](int sc) {
        if constexpr (kAcc)
            pacc = bload4<float>(make_rsrc_in(p.acc, acc_off, p.acc_in_end), oacc, uint32_t(sc * kSC) * 4u);
    };

    // out / y of super-chunk sc (its 64 sums are in yo); `real` false: the
    // placeholder call of a segment's first super-chunk, whose out / y stores
    // the real call rewrites later and whose accumulator store is dropped (a
    // middle pass reads the accumulator in place, right after this call)
    auto finish_super = [&](int sc, bool real) {
        float4 y = *reinterpret_cast<const float4*>(yo + 4 * r);
        if constexpr (kAcc) {
            y.x += pacc.x; y.y += pacc.y; y.z += pacc.z; y.w += pacc.w;
            bstore4<float, kStoreNT>(
                make_rsrc_in(p.acc, acc_off + int64_t(sc) * kSC * 4, real ? p.acc_out_end : 0), oacc, y);
        }
        y.x = __builtin_fmaf(Dv, pu.x, y.x);
        y.y = __builtin_fmaf(Dv, pu.y, y.y);
        y.z = __builtin_fmaf(Dv, pu.z, y.z);
        y.w = __builtin_fmaf(Dv, pu.w, y.w);
        // (non-temporal out / y stores only for 16-byte aligned rows, see
        // FwdParams::store_nt; the branch is uniform)
        if constexpr (kZ) {
            const rsrc_t Ry = make_rsrc_in(p.y, y_off + int64_t(sc) * kSC * es64, y_end);
            if (p.store_nt) bstore4<IT, kStoreNT>(Ry, oy, y);
            else bstore4<IT, kStoreDefault>(Ry, oy, y);
            y.x *= pz.x * sigmoidf_(pz.x);
            y.y *= pz.y * sigmoidf_(pz.y);
            y.z *= pz.z * sigmoidf_(pz.z);
            y.w *= pz.w * sigmoidf_(pz.w);
        }
        const rsrc_t Ro = make_rsrc_in(p.out, o_off + int64_t(sc) * kSC * es64, p.o_end);
        if (p.store_nt) bstore4<IT, kStoreNT>(Ro, oo, y);
        else bstore4<IT, kStoreDefault>(Ro, oo, y);
    };
    // as finish_super for the tail super-chunk: element stores of its lt steps
    auto finish_super_tail = [&](int sc) {
        float4 y = *reinterpret_cast<const float4*>(yo + 4 * r);
        if constexpr (kAcc) {
            y.x += pacc.x; y.y += pacc.y; y.z += pacc.z; y.w += pacc.w;
            const rsrc_t Ra = make_rsrc_in(p.acc, acc_off + int64_t(sc) * kSC * 4, p.acc_out_end);
            const float av[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (4 * r + i < lt) bstore<float, kStoreNT>(Ra, oacc + uint32_t(i) * 4u, 0, av[i]);
        }
        y.x = __builtin_fmaf(Dv, pu.x, y.x);
        y.y = __builtin_fmaf(Dv, pu.y, y.y);
        y.z = __builtin_fmaf(Dv, pu.z, y.z);
        y.w = __builtin_fmaf(Dv, pu.w, y.w);
        float yv[4] = {y.x, y.y, y.z, y.w}, zv[4] = {pz.x, pz.y, pz.z, pz.w};
        const rsrc_t Ro = make_rsrc_in(p.out, o_off + int64_t(sc) * kSC * es64, p.o_end);
        const rsrc_t Ryt = make_rsrc_in(p.y, y_off + int64_t(sc) * kSC * es64, y_end);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (4 * r + i < lt) {
                float o = yv[i];
                if constexpr (kZ) {
                    bstore<IT, kStoreDefault>(Ryt, oy + uint32_t(i) * es, 0, o);
                    o *= zv[i] * sigmoidf_(zv[i]);
                }
                bstore<IT, kStoreDefault>(Ro, oo + uint32_t(i) * es, 0, o);
            }
        }
    };
    // y_t = sum over states of C h for the chunk whose states are in the
    // tile: lane r reads step r's 16 states, and multiplies them by that
    // step's C row (read from the transposed tile while the chunk ran)
    auto read_tile = [&](float (&ys)[kT]) {
#pragma unroll
        for (int n = 0; n < kT; ++n) ys[n] = yrow[n * 16 + yoff[(n >> 1) & 3]];
    };
    auto dot16 = [&](const float (&ys)[kT], const float (&cv)[kT]) {
        float s0 = ys[0] * cv[0], s1 = ys[1] * cv[1];
#pragma unroll
        for (int n = 2; n < kT; n += 2) {
            s0 = __builtin_fmaf(ys[n], cv[n], s0);
            s1 = __builtin_fmaf(ys[n + 1], cv[n + 1], s1);
        }
        return s0 + s1;
    };
    // C of step r of the chunk last run, states 0..15 (constant C: the 16 C
    // of this lane's channel, for every step)
    float cT[kT];
#pragma unroll
    for (int n = 0; n < kT; ++n) cT[n] = kVC ? 0.f : static_cast<const float*>(p.C)[c * p.C_gs + n * p.C_ns];

    Super S;
    // one super-chunk: the full ones prefetch the next and stage its B / C
    // tile; the tail (TAIL) zeroes the decay exponents and inputs of the steps
    // past the sequence (identity steps: a = 1, b = 0) and drops the
    // checkpoints of chunks past it
    auto super_chunk = [&](int sc, auto TAIL) {
        constexpr bool kTail = decltype(TAIL)::value;
        const int buf = (sc - sc0) & 1;
        if constexpr (kVB || kVC) lds_barrier();   // B / C tile of sc staged (the other LDS areas are per row)
        const float4 cu = S.u, cd = S.d, cz = S.z;
        if constexpr (!kTail) fetch(sc + 1 < scf ? sc + 1 : scf - 1, S);

        float4 dt, dtu;
        {
            const float p0 = cd.x + bias, p1 = cd.y + bias, p2 = cd.z + bias, p3 = cd.w + bias;
            dt = softplus ? make_float4(softplus20(p0), softplus20(p1), softplus20(p2), softplus20(p3))
                          : make_float4(p0, p1, p2, p3);
            dtu = make_float4(dt.x * cu.x, dt.y * cu.y, dt.z * cu.z, dt.w * cu.w);
            if constexpr (kTail) {
                dt.x = 4 * r + 0 < lt ? dt.x : 0.f;
                dt.y = 4 * r + 1 < lt ? dt.y : 0.f;
                dt.z = 4 * r + 2 < lt ? dt.z : 0.f;
                dt.w = 4 * r + 3 < lt ? dt.w : 0.f;
            }
        }
        dpp_sources_ready4(dt, dtu);
        if (sc >= x_w0 + x_wsc) {
            x_w0 = sc;
            Rx_w = make_rsrc_in(p.x, x_off + int64_t(kQ * sc) * x_chunk_bytes, p.x_end);
            Rx_wt = make_rsrc_in(p.x, x_off + int64_t(kQ * sc) * x_chunk_bytes, x_tail_end);
        }
        const rsrc_t Rx = kTail ? Rx_wt : Rx_w;
        const uint32_t x_so = uint32_t((sc - x_w0) * kQ) * uint32_t(x_chunk_bytes);
        const float* sB = s_bc + (buf * 2 + 0) * 16 * kSC;
        const float* sC = s_bc + (buf * 2 + 1) * 16 * kSC;

        static_for<kQ>([&](auto Q) {
            constexpr int q = decltype(Q)::value;
            // B of this lane's state for the chunk's 16 steps (read here, or
            // just before the recurrence for the 128-VGPR build)
            float Bq[kT];
            if constexpr (!fwd_late_b<IT, kAcc>()) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if constexpr (kVB) {
                        const float4 vb = *reinterpret_cast<const float4*>(sB + bc64_slot(r, 4 * q + i));
                        Bq[4 * i] = vb.x; Bq[4 * i + 1] = vb.y; Bq[4 * i + 2] = vb.z; Bq[4 * i + 3] = vb.w;
                    } else {
                        Bq[4 * i] = Bq[4 * i + 1] = Bq[4 * i + 2] = Bq[4 * i + 3] = bconst;
                    }
                }
            }
            // states of the previous chunk, written by this row last chunk
            float ys[kT];
            read_tile(ys);
            // decay factors of all 16 steps first: they do not depend on h, so
            // the exp latency stays off the h chain
            float a[kT];
            static_for<kT>([&](auto K) {
                constexpr int k = decltype(K)::value;
                a[k] = __builtin_amdgcn_exp2f(row_bcast<4 * q + k / 4>(f4get(dt, k % 4)) * a2);
            });
            // the LDS reads issued above have had the decay factors to land
            __builtin_amdgcn_sched_barrier(0);
            // the previous chunk's sums (chunk 4 sc + q - 1) into the regroup area
            yo[((q + kQ - 1) % kQ) * kT + r] = dot16(ys, cT);
            if constexpr (q == 0) {
                if constexpr (kTail) {
                    if (sc > sc0) finish_super(sc - 1, true);
                    acc_load(sc);
                } else {
                    finish_super(sc > sc0 ? sc - 1 : sc0, sc > sc0);   // (at sc0 a placeholder, rewritten later)
                    acc_load(sc);
                }
                pu = cu;     // this super-chunk's u, z wait for its outputs
                pz = cz;
            }
            if constexpr (fwd_late_b<IT, kAcc>()) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if constexpr (kVB) {
                        const float4 vb = *reinterpret_cast<const float4*>(sB + bc64_slot(r, 4 * q + i));
                        Bq[4 * i] = vb.x; Bq[4 * i + 1] = vb.y; Bq[4 * i + 2] = vb.z; Bq[4 * i + 3] = vb.w;
                    } else {
                        Bq[4 * i] = Bq[4 * i + 1] = Bq[4 * i + 2] = Bq[4 * i + 3] = bconst;
                    }
                }
            }
            float yp[kT];
            static_for<kT>([&](auto K) {
                constexpr int k = decltype(K)::value;
                h = __builtin_fmaf(a[k], h, bmul<4 * q + k / 4>(f4get(dtu, k % 4), Bq[k]));
                yp[k] = h;
            });
            bstore<float, kStoreNT>(Rx, ox, x_so + uint32_t(q * x_chunk_bytes), h);
#pragma unroll
            for (int m = 0; m < 4; ++m)
                *reinterpret_cast<float4*>(yrow + r * 16 + 4 * (m ^ ((r >> 1) & 3))) =
                    make_float4(yp[4 * m], yp[4 * m + 1], yp[4 * m + 2], yp[4 * m + 3]);
            // C of step r of this chunk, for its sum one chunk later (read
            // now: this buffer is not restaged before the next barrier)
            if constexpr (kVC) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float4 vc = *reinterpret_cast<const float4*>(sC + ct_slot4(16 * q + r, i));
                    cT[4 * i] = vc.x; cT[4 * i + 1] = vc.y; cT[4 * i + 2] = vc.z; cT[4 * i + 3] = vc.w;
                }
            }
        });
        // B / C tile of the next super-chunk into the other buffer
        if constexpr (!kTail) stage(S, buf ^ 1);
    };
    if (scf > sc0) {
        fetch(sc0, S);
        stage(S, 0);
    }
    for (int sc = sc0; sc < scf; ++sc) super_chunk(sc, std::false_type{});
    if (tail) {
        fetch_tail(scf, S);
        stage(S, (scf - sc0) & 1);
        super_chunk(scf, std::true_type{});
    }
    // the last chunk's sums, then the last super-chunk's outputs
    {
        float ys[kT];
        read_tile(ys);
        yo[(kQ - 1) * kT + r] = dot16(ys, cT);
        if (tail) finish_super_tail(sc1 - 1);
        else finish_super(sc1 - 1, true);
    }
    if (p.last_state && seg == nseg - 1) p.last_state[(b * p.dim + c) * xN + r] = h;
}

// Pass A of the sequence-parallel forward: workgroup (b, seg, 16 channels)
// scans segment seg (nseg - 1 of them: the last segment's end state is not
// needed) from a zero state with the fast kernel's lane layout and
// arithmetic, but only the state recurrence (no C, no outputs), and writes
// the state after the segment's last step to seg_h and the segment's sum of
// delta' to seg_s.  About three fifths of a full scan's work per step.
// kVB false: B constant ((dim, dstate) fp32, in a register; no tile, no
// barrier).
template <typename IT, bool kVB>
__global__ __launch_bounds__(kThreads, 3) void ss_fwd_seg_state(const FwdParams p) {
    __shared__ __attribute__((aligned(16))) float s_b[2 * 16 * kSC];               // [buf][n][64 steps]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int r = lane & 15;
    const int j = lane >> 4;
    const int row = w * kRows + j;
    const int64_t nblk = p.dim / kChPerWG;
    const int nsa = p.nseg - 1;                    // segments scanned here
    const int64_t blk = xcd_block_id();
    const int64_t bs = blk / nblk;
    const int64_t b = bs / nsa;
    const int seg = int(bs % nsa);
    const int64_t c0 = (blk % nblk) * kChPerWG;
    const int64_t c = c0 + row;
    const int64_t g = c0 / p.dpg;
    // segments 0 .. nseg - 2 only: whole super-chunks (the tail ends the last)
    const int nsc_pad = int((p.seqlen + kSC - 1) / kSC);
    const int sc0 = seg_begin(seg, nsc_pad, p.nseg), sc1 = seg_begin(seg + 1, nsc_pad, p.nseg);

    constexpr int64_t es64 = sizeof(IT);
    const rsrc_t Ru = make_rsrc_in(p.u, (b * p.u_bs + c0 * p.u_ds) * es64, p.u_end);
    const rsrc_t Rd = make_rsrc_in(p.delta, (b * p.dl_bs + c0 * p.dl_ds) * es64, p.dl_end);
    const rsrc_t RB = kVB ? make_rsrc_in(p.B, (b * p.B_bs + g * p.B_gs) * es64, p.B_end) : make_rsrc_n(nullptr, 0);
    constexpr uint32_t es = sizeof(IT);
    const uint32_t ou = uint32_t(row * p.u_ds + 4 * r) * es, od = uint32_t(row * p.dl_ds + 4 * r) * es;
    const uint32_t oB = uint32_t(row * p.B_ns + 4 * r) * es;

    const float bias = p.delta_bias ? p.delta_bias[c] : 0.f;
    const float a2 = p.A[c * p.A_ds + r * p.A_ns] * kLog2e;
    const bool softplus = p.softplus != 0;
    const float bconst = kVB ? 0.f : static_cast<const float*>(p.B)[c * p.B_gs + r * p.B_ns];

    struct Seg { float4 u, d, B; };
    auto fetch = [&](int sc, Seg& S) {
        const uint32_t so = uint32_t(sc * kSC) * es;
        S.u = bload4<IT>(Ru, ou, so);
        S.d = bload4<IT>(Rd, od, so);
        S.B = kVB ? bload4<IT>(RB, oB, so) : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    auto stage = [&](const Seg& S, int buf) {
        if constexpr (kVB) *reinterpret_cast<float4*>(s_b + buf * 16 * kSC + bc64_slot(row, r)) = S.B;
    };

    float h = 0.f, dsum = 0.f;
    Seg S;
    fetch(sc0, S);
    stage(S, 0);
    for (int sc = sc0; sc < sc1; ++sc) {
        const int buf = (sc - sc0) & 1;
        if constexpr (kVB) lds_barrier();   // B tile of sc staged
        const float4 cu = S.u, cd = S.d;
        fetch(sc + 1 < sc1 ? sc + 1 : sc1 - 1, S);
        float4 dt, dtu;
        {
            const float p0 = cd.x + bias, p1 = cd.y + bias, p2 = cd.z + bias, p3 = cd.w + bias;
            dt = softplus ? make_float4(softplus20(p0), softplus20(p1), softplus20(p2), softplus20(p3))
                          : make_float4(p0, p1, p2, p3);
            dtu = make_float4(dt.x * cu.x, dt.y * cu.y, dt.z * cu.z, dt.w * cu.w);
        }
        dsum += (dt.x + dt.y) + (dt.z + dt.w);
        dpp_sources_ready4(dt, dtu);
        const float* sB = s_b + buf * 16 * kSC;
        static_for<kQ>([&](auto Q) {
            constexpr int q = decltype(Q)::value;
            float Bq[kT];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (kVB) {
                    const float4 vb = *reinterpret_cast<const float4*>(sB + bc64_slot(r, 4 * q + i));
                    Bq[4 * i] = vb.x; Bq[4 * i + 1] = vb.y; Bq[4 * i + 2] = vb.z; Bq[4 * i + 3] = vb.w;
                } else {
                    Bq[4 * i] = Bq[4 * i + 1] = Bq[4 * i + 2] = Bq[4 * i + 3] = bconst;
                }
            }
            // the recurrence at raised wave priority (unlike the full forward;
            // 1 x 1536 x 32768 bf16 forward with segments 422 -> 408 us)
            __builtin_amdgcn_s_setprio(1);
            float a[kT];
            static_for<kT>([&](auto K) {
                constexpr int k = decltype(K)::value;
                a[k] = __builtin_amdgcn_exp2f(row_bcast<4 * q + k / 4>(f4get(dt, k % 4)) * a2);
            });
            static_for<kT>([&](auto K) {
                constexpr int k = decltype(K)::value;
                h = __builtin_fmaf(a[k], h, bmul<4 * q + k / 4>(f4get(dtu, k % 4), Bq[k]));
            });
        });
        __builtin_amdgcn_s_setprio(0);
        stage(S, buf ^ 1);
    }
    const int64_t si = (b * p.nseg + seg) * p.dim + c;
    p.seg_h[si * kT + r] = h;
    dsum = row_allsum(dsum);                       // the row's 16 lanes hold 4 steps each
    if (r == 0) p.seg_s[si] = dsum;
}

// Segments for the forward (seg_count): at least kSegMinSC super-chunks
// each; 1 (serial) when the fast path does not apply.
bool fwd_fast_ok(const FwdParams& p);
constexpr int kSegMinSC = 4;
int fwd_segments(const FwdParams& p) {
    if (!fwd_fast_ok(p)) return 1;
    return seg_count(p.batch * (p.dim / kChPerWG), (p.seqlen + kSC - 1) / kSC, kSegMinSC);
}

bool fwd_fast_ok(const FwdParams& p) {
    // every byte offset the kernel forms stays below 2^32: rows and seqlen
    // below 2^26 elements, checkpoints addressed from each super-chunk's
    // first chunk (dim x the checkpoints' states per channel below 2^28)
    // (a seqlen that is not a multiple of 64 ends in a partial super-chunk)
    return p.dstate == 16 && p.seqlen >= 1 &&
           p.dim % kChPerWG == 0 && p.dpg % kChPerWG == 0 &&
           small_strides({p.seqlen, p.u_ds, p.dl_ds, p.z_ds, p.o_ds, p.y_ds, p.B_ns, p.C_ns}) &&
           p.dim * p.xN < (int64_t(1) << 28);
}

// the fast forward for the combination of variable / constant B and C
template <typename IT, bool kZ>
static void launch_fwd_bc(const FwdParams& p, dim3 grid, dim3 block, hipStream_t stream) {
    if (p.var_B && p.var_C) hipLaunchKernelGGL((ss_fwd_fast<IT, kZ, false, true, true>), grid, block, 0, stream, p);
    else if (p.var_B) hipLaunchKernelGGL((ss_fwd_fast<IT, kZ, false, true, false>), grid, block, 0, stream, p);
    else if (p.var_C) hipLaunchKernelGGL((ss_fwd_fast<IT, kZ, false, false, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((ss_fwd_fast<IT, kZ, false, false, false>), grid, block, 0, stream, p);
}

template <typename IT>
static hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
    const int64_t nblk = (p.dim + kChPerWG - 1) / kChPerWG;
    const dim3 grid(unsigned(nblk * p.batch));
    const dim3 block(kThreads);
    const int spl = int((p.dstate + 15) / 16);
    const bool vbc = p.var_B && p.var_C;
    if (fwd_fast_ok(p)) {
        const int nseg = p.nseg > 1 ? p.nseg : 1;
        if (nseg > 1) {
            const dim3 agrid(unsigned(nblk * p.batch * (nseg - 1)));
            if (p.var_B) hipLaunchKernelGGL((ss_fwd_seg_state<IT, true>), agrid, block, 0, stream, p);
            else hipLaunchKernelGGL((ss_fwd_seg_state<IT, false>), agrid, block, 0, stream, p);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        const dim3 sgrid(unsigned(nblk * p.batch * nseg));
        if (p.acc) {
            if (p.has_z) hipLaunchKernelGGL((ss_fwd_fast<IT, true, true, true, true>), sgrid, block, 0, stream, p);
            else hipLaunchKernelGGL((ss_fwd_fast<IT, false, true, true, true>), sgrid, block, 0, stream, p);
        } else if (p.has_z) {
            launch_fwd_bc<IT, true>(p, sgrid, block, stream);
        } else {
            launch_fwd_bc<IT, false>(p, sgrid, block, stream);
        }
    } else if (spl <= 1) {
        if (vbc) hipLaunchKernelGGL((ss_fwd_kernel<IT, 1, true>), grid, block, 0, stream, p);
        else hipLaunchKernelGGL((ss_fwd_kernel<IT, 1, false>), grid, block, 0, stream, p);
    } else if (spl <= 2) hipLaunchKernelGGL((ss_fwd_kernel<IT, 2, false>), grid, block, 0, stream, p);
    else if (spl <= 4) hipLaunchKernelGGL((ss_fwd_kernel<IT, 4, false>), grid, block, 0, stream, p);
    else if (spl <= 8) hipLaunchKernelGGL((ss_fwd_kernel<IT, 8, false>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((ss_fwd_kernel<IT, 16, false>), grid, block, 0, stream, p);
    return hipGetLastError();
}

const char* fwd_kernel_name(const FwdParams& p) { return fwd_fast_ok(p) ? "ss_fwd_fast" : "ss_fwd_kernel"; }

hipError_t launch_fwd(const FwdParams& p, int itype, hipStream_t stream) {
    switch (itype) {
        case SS_F32: return launch_fwd_t<float>(p, stream);
        case SS_BF16: return launch_fwd_t<bf16_t>(p, stream);
        case SS_F16: return launch_fwd_t<_Float16>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace ss
