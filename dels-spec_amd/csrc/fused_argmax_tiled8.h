// fp8 (e4m3) variant of the MFMA-tiled fused combine + vocabulary argmax, for
// many rows (M >= 64): B in e4m3 K128 blocks with per-row fp32 scales, the
// rank quantised per row to e4m3 beforehand (quantize_rank_e4m3_kernel: bytes
// [M][r] and one scale per row, read here as the MFMA operand; quantising in
// this kernel's prologue spilled), v_mfma_scale_f32_32x32x64_f8f6f4.
//
// Per row m and vocabulary row v (the fp8 GEMV's semantics):
//     dot      = f32(f32(acc[m, v] * sR[m]) * sB[v])      acc: the e4m3 x e4m3 contraction
//     s[m, v]  = dot * alpha_m + base[m, v] - beta_m * prior[v]   (two fused multiply-adds)
// and per row the lowest v attaining the maximum.  The rank quantisation is
// the GEMV's: amax = max |rank[m, :]|, inv = 448 / amax, q = e4m3(rank * inv),
// sR = amax / 448 (1 and zeros for an all-zero row).
//
// The structure is the bf16 tiled kernel's (fused_argmax_tiled.h): 8 waves of
// 32 rows, 256 rows and a contiguous chunk of 32-column vocabulary tiles per
// workgroup, one tile per stage, B in LDS by direct-to-LDS loads, the base
// logits in whole 128-byte lines per row (a two-chunk ring),
// the vocabulary rows of a tile permuted so that each lane holds 16 consecutive
// columns, the combine of stage st-1 interleaved between the MFMAs of stage st.
// What differs is the operand order: the 32x32x64 MFMA takes, for lane l, 32
// consecutive K bytes 32*(l/32) .. of row l%32 of a 64-deep step.  The K128
// blocks (16 rows x 128 K, lane L: row L%16, K 32*(L/16) .. +31 as two 16-byte
// halves) hold exactly those runs, so the B tile is gathered into step-major
// LDS blocks of 2 KiB ([half][lane][16 B]) by the loads themselves; every
// operand read is then two contiguous KiB.  The rank operand uses the same K
// order (bytes in natural order within each 32-byte run), so the MFMA, which
// pairs A and B by (lane group, byte), computes the plain dot product.  B is
// half the bytes of the bf16 kernel's, so the base logits are most of what the
// CUs take in -- and the LDS holds three B tiles (with 16-bit base logits),
// the tile of stage st + 2 loading while st is contracted (M=512 step 80.6 ->
// 79.2 us against two).
#pragma once

#include "fp8.h"
#include "fused_argmax_tiled.h"

namespace dels {

namespace tiled8 {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kTileCols = 32;
constexpr int kSideBytes = 256;   // per wave and stage: the prior slice, the B scales
constexpr int kOperandAhead = 2;

// 64-deep K steps of r = 128 * KS8.
template <int KS8>
constexpr int steps() { return 2 * KS8; }

__device__ __forceinline__ f32x16 mfma_e4m3_32x32x64(const i32x8& a, const i32x8& b, f32x16 acc) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc, 0, 0, 0, 127, 0, 127);
}

}  // namespace tiled8

// EXACT: V is a multiple of the 32-column tile, so no tile needs masking.
template <int KS8, typename BaseT, typename PriorT, bool EXACT>
__global__ __launch_bounds__(tiled8::kThreads) void fused_argmax_tiled8_kernel(TiledKArgs a) {
#pragma clang fp contract(off)
    using namespace tiled8;
    using tiled::kLineBytes;
    using tiled::kRowsPerWG;
    constexpr int kSteps = steps<KS8>();                             // 64-deep K steps
    constexpr bool kPrior = !is_no_prior<PriorT>::value;
    constexpr int SPC = tiled::stages_per_chunk<BaseT>();            // 2 (16-bit base) or 1 (fp32)
    constexpr int kBPieces = 2 * kSteps / kWaves;                    // 1-KiB B loads per wave and stage
    constexpr int kQPieces = kRowsPerWG * kLineBytes / 1024 / kWaves; // base chunk loads per wave (4)
    constexpr int kEB = kBPieces + 1 + (kPrior ? 1 : 0);              // + the B scales, + the prior
    constexpr int kWB = sizeof(BaseT) == 4 ? 16 : 8;
    constexpr int kWP = sizeof(PriorT) == 4 ? 16 : 8;
    constexpr int kCands = 16;
    constexpr int kAhead = kOperandAhead;
    static_assert((2 * kSteps) % kWaves == 0, "B loads per stage must split over the waves");

    struct __attribute__((aligned(1024))) BBuf {
        char b[kSteps * 2048];                   // [step][half][lane][16 B]
        char prior[kWaves][kSideBytes];
        char bsc[kWaves][kSideBytes];            // fp32 scales of the tile's 32 vocabulary rows
    };
    struct __attribute__((aligned(1024))) QBuf {
        char q[kRowsPerWG * kLineBytes];         // one 128-byte line of base logits per row
    };
    // B tiles: with 16-bit base logits three buffers, the loads of stage st + 2
    // in flight while st is contracted; with fp32 ones (a base chunk per stage,
    // loaded one stage ahead) two
    constexpr int kNB = SPC == 2 ? 3 : 2;
    __shared__ BBuf bb[kNB];
    __shared__ QBuf qb0, qb1;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rl = lane & 31;
    const int h = lane >> 5;
    const int m_wg = blockIdx.y * kRowsPerWG;
    const int mw = m_wg + wave * 32;
    const bool wave_active = mw < a.M;
    // vocabulary chunk: tiles [T0, T0 + nst), starting on a base chunk boundary
    const int nunits = (a.ntiles + SPC - 1) / SPC;
    const int u0 = (int)(((int64_t)blockIdx.x * nunits) / gridDim.x);
    const int u1 = (int)(((int64_t)(blockIdx.x + 1) * nunits) / gridDim.x);
    const int T0 = u0 * SPC;
    const int nst = max(0, min(a.ntiles, u1 * SPC) - T0);
    const int last_chunk = max(nst - 1, 0) / SPC;
    auto tile_of = [&](int st) { return min(T0 + min(st, max(nst - 1, 0)), a.ntiles - 1); };

    // ---- the rank operand: this lane's row, K runs 64s + 32h .. +31, e4m3 ----
    // (quantised beforehand: rank_q [M][ldrank] bytes, sR [M])
    const int mrow = min(mw + rl, a.M - 1);
    const uint8_t* rqp = a.rank_q + (int64_t)mrow * a.ldrank + 32 * h;
    i32x8 rq[kSteps];
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        const u32x4 lo = *reinterpret_cast<const u32x4*>(rqp + 64 * s);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(rqp + 64 * s + 16);
        rq[s] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
    const float sR = a.rank_scale[mrow];
    const float al = a.alpha[(int64_t)mrow * a.alpha_stride];
    const float be = a.beta[(int64_t)mrow * a.beta_stride];
    // beta == 0 skips the prior term: fma(0, +0, sc) == sc, whatever the prior holds
    const bool use_prior = kPrior && be != 0.f;
    const float nbeta = use_prior ? -be : 0.f;
    const uint32_t pmask = use_prior ? 0xffffffffu : 0u, pmask_hi = use_prior ? 0xffff0000u : 0u;
    const uint32_t psel_lo = use_prior ? 0x01000c0cu : 0x0c0c0c0cu;   // v_perm_b32: bytes 1,0 -> 3,2
    float best = -__builtin_inff();
    int bidx = INT_MAX;
    // Drain the loads above before any direct-to-LDS load (see the bf16 kernel:
    // otherwise the compiler waits for every stage load before each MFMA).
    __builtin_amdgcn_s_waitcnt(0x0070 | (0xf << 8));   // vmcnt(0)

    const char* Bg = reinterpret_cast<const char*>(a.B);
    const char* priorg = static_cast<const char*>(a.prior);
    const char* bscg = reinterpret_cast<const char*>(a.b_scale);

    // B gather: load (step s, half h2) puts, in MFMA lane l, 16 bytes of the K128
    // block (block row 2T + perm_block(l%32), K block s/2), lane perm_row(l%32) +
    // 16*(2*(s%2) + l/32), half h2 -- the 32 vocabulary rows permuted as in the
    // bf16 kernel, so that lane l ends with the columns 16h .. 16h+15.
    const int hh = tiled::perm_block(rl);
    const uint32_t b_lane = (uint32_t)(tiled::perm_row(rl) * 16 + h * 256);
    auto issue_b = [&](BBuf& S, int st, int piece) {
        const int blk = min(2 * tile_of(st) + hh, a.nblk16 - 1);
        const int ii = wave * kBPieces + piece;            // (step, half) of this load
        const int s = ii >> 1, h2 = ii & 1;
        const uint32_t off = (uint32_t)blk * (uint32_t)(KS8 * kFp8K128Block) + (uint32_t)(s >> 1) * kFp8K128Block +
                             (uint32_t)(s & 1) * 512 + (uint32_t)h2 * 1024 + b_lane;
        dma16(Bg, off, S.b + s * 2048 + h2 * 1024);
    };
    auto issue_side = [&](BBuf& S, int st, int which) {   // 0: B scales, 1: prior
        const int vs = tile_of(st) * kTileCols;
        if (which == 0) {
            dma4(bscg, (uint32_t)min(vs + (lane & 31), a.V - 1) * 4u, S.bsc[wave]);
        } else if constexpr (kPrior) {
            if constexpr (sizeof(PriorT) == 4) dma4(priorg, (uint32_t)min(vs + (lane & 31), a.V - 1) * 4u, S.prior[wave]);
            else dma4(priorg, (uint32_t)min(vs + 2 * (lane & 15), a.V - 2) * 2u, S.prior[wave]);
        }
    };
    auto issue_q = [&](QBuf& Q, int c, int piece) {
        tiled::dma_base_lines<BaseT>(a, m_wg, (T0 + min(c, last_chunk) * SPC) * kTileCols, wave * kQPieces + piece,
                                     Q.q);
    };
    // Loads of the next stage: B, the B scales and the prior of st + 1, then (the
    // stages that open a chunk) base chunk c_next -- last, so that a wait for B can
    // leave it in flight.
    auto issue_piece = [&](BBuf& S, int st_next, QBuf& Q, int c_next, int piece) {
        if (piece < kBPieces) issue_b(S, st_next, piece);
        else if (piece < kEB) issue_side(S, st_next, piece - kBPieces);
        else issue_q(Q, c_next, piece - kEB);
    };

    // Epilogue operands of one stage in registers (candidate j is the lane's
    // column 16h + j): base, prior and B scale values; columns past V carry a
    // -inf base.
    struct EpiRegs {
        uint32_t b[kWB];
        uint32_t p[kWP];
        float sb[16];
    };
    constexpr uint32_t kNegInf = sizeof(BaseT) == 4 ? 0xff800000u : tiled::half_neg_inf<BaseT>();
    const int qrow = wave * 32 + rl;
    auto load_epi_group = [&](const QBuf& Q, const BBuf& S, int st, int g, EpiRegs& e) {
        const int vs = tile_of(st) * kTileCols;
        const int v = vs + 16 * h + 4 * g;
        const bool partial = !EXACT && vs + kTileCols > a.V;
        const char* src = tiled::line_at(Q.q, qrow, ((st % SPC) * kTileCols + 16 * h + 4 * g) * (int)sizeof(BaseT));
        if constexpr (sizeof(BaseT) == 4) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(src);
#pragma unroll
            for (int q = 0; q < 4; ++q) e.b[4 * g + q] = (partial && v + q >= a.V) ? kNegInf : w[q];
        } else {
            const uint2 w = *reinterpret_cast<const uint2*>(src);
            uint32_t w0 = w.x, w1 = w.y;
            if (partial) {
                w0 = v < a.V ? w0 : ((w0 & 0xffff0000u) | kNegInf);
                w0 = v + 1 < a.V ? w0 : ((w0 & 0xffffu) | (kNegInf << 16));
                w1 = v + 2 < a.V ? w1 : ((w1 & 0xffff0000u) | kNegInf);
                w1 = v + 3 < a.V ? w1 : ((w1 & 0xffffu) | (kNegInf << 16));
            }
            e.b[2 * g] = w0;
            e.b[2 * g + 1] = w1;
        }
        const f32x4 sv = *reinterpret_cast<const f32x4*>(S.bsc[wave] + (16 * h + 4 * g) * 4);
#pragma unroll
        for (int q = 0; q < 4; ++q) e.sb[4 * g + q] = sv[q];
        if constexpr (kPrior) {
            const char* pp = S.prior[wave] + (16 * h + 4 * g) * (int)sizeof(PriorT);
            if constexpr (sizeof(PriorT) == 4) {
                const u32x4 w = *reinterpret_cast<const u32x4*>(pp);
#pragma unroll
                for (int q = 0; q < 4; ++q) e.p[4 * g + q] = w[q];
            } else {
                const uint2 w = *reinterpret_cast<const uint2*>(pp);
                e.p[2 * g] = w.x;
                e.p[2 * g + 1] = w.y;
            }
        }
    };
    // Candidate j of the previous stage (first column cb); the empty volatile asm
    // statements pin its work between the MFMAs (pure arithmetic would otherwise
    // be gathered after the last MFMA of the stage).
    auto epi_one = [&](const f32x16& accp, const EpiRegs& e, int cb, int j) {
        float av = accp[j];
        float sbv = e.sb[j];
        const uint32_t bw = e.b[sizeof(BaseT) == 4 ? j : (j >> 1)];
        float bv = sizeof(BaseT) == 4 ? __uint_as_float(bw) : tiled::half_at<BaseT>(bw, j & 1);
        asm volatile("" : "+v"(av), "+v"(sbv), "+v"(bv));
        float dot = av * sR;
        dot = dot * sbv;
        float sc = __builtin_fmaf(dot, al, bv);
        if constexpr (kPrior) {
            const uint32_t pw = e.p[sizeof(PriorT) == 4 ? j : (j >> 1)];
            float pv;   // the prior value, or +0 for a row without the prior term
            if constexpr (sizeof(PriorT) == 4) pv = __uint_as_float(pw & pmask);
            else if constexpr (std::is_same<PriorT, bf16_t>::value)
                pv = __uint_as_float((j & 1) ? (pw & pmask_hi) : __builtin_amdgcn_perm(pw, pw, psel_lo));
            else pv = __uint_as_float(__float_as_uint(tiled::half_at<PriorT>(pw, j & 1)) & pmask);
            asm volatile("" : "+v"(pv));
            sc = __builtin_fmaf(nbeta, pv, sc);
        }
        const bool take = sc > best;   // candidates arrive in increasing index order
        best = take ? sc : best;
        bidx = take ? cb + j : bidx;
        asm volatile("" : "+v"(best), "+v"(bidx));
    };
    constexpr int kPer = (kCands + kSteps - 1) / kSteps;   // candidates per MFMA slot
    // Sn receives the B tile of stage st + kNB - 1.
    auto contract = [&](auto issue_q_tag, const BBuf& S, const QBuf& Q, int st, BBuf& Sn, QBuf& Qn, int c_next,
                        f32x16& acc, const f32x16& accp, const EpiRegs& ep, int cbp, EpiRegs& epn) {
        constexpr bool ISSUE_Q = decltype(issue_q_tag)::value;
        constexpr int E = kEB + (ISSUE_Q ? kQPieces : 0);
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.f;
        auto opnd = [&](int s) {
            const u32x4 lo = *reinterpret_cast<const u32x4*>(S.b + s * 2048 + lane * 16);
            const u32x4 hi = *reinterpret_cast<const u32x4*>(S.b + s * 2048 + 1024 + lane * 16);
            return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2],
                         (int)hi[3]};
        };
        i32x8 opq[kAhead];
#pragma unroll
        for (int i = 0; i < kAhead; ++i) opq[i] = opnd(i < kSteps ? i : 0);
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const i32x8 a0 = opq[s % kAhead];
            if (s + kAhead < kSteps) opq[s % kAhead] = opnd(s + kAhead);
            __builtin_amdgcn_sched_barrier(0);
            acc = mfma_e4m3_32x32x64(a0, rq[s], acc);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int c = s * kPer; c < (s + 1) * kPer && c < kCands; ++c) {
                epi_one(accp, ep, cbp, c);
                if ((c & 3) == 3) load_epi_group(Q, S, st, c >> 2, epn);
            }
#pragma unroll
            for (int piece = 0; piece < E; ++piece)
                if (s == piece * kSteps / E) issue_piece(Sn, st + kNB - 1, Qn, c_next, piece);
        }
        // candidates not reached in the loop (fewer slots than 16 / kPer)
#pragma unroll
        for (int c = kSteps * kPer; c < kCands; ++c) {
            epi_one(accp, ep, cbp, c);
            if ((c & 3) == 3) load_epi_group(Q, S, st, c >> 2, epn);
        }
    };
    auto issue_all = [&](auto issue_q_tag, BBuf& Sn, int st_next, QBuf& Qn, int c_next) {
        constexpr int E = kEB + (decltype(issue_q_tag)::value ? kQPieces : 0);
#pragma unroll
        for (int piece = 0; piece < E; ++piece) issue_piece(Sn, st_next, Qn, c_next, piece);
    };

    // Pipeline as the bf16 kernel's: B(0), its side slices and base chunk 0 up
    // front; at stage st every wave waits for its own loads of B(st) (the chunk
    // loads issued during an even stage may stay in flight through the next
    // barrier), the barrier publishes st, and the loads of st + 1 (and of the
    // next chunk when st opens one) go out while st is contracted.
    f32x16 acc_prev;
    EpiRegs ep_prev, ep_cur;
    int cb_prev = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        acc_prev[i] = 0.f;
        ep_prev.sb[i] = 1.f;
    }
#pragma unroll
    for (int i = 0; i < kWB; ++i) ep_prev.b[i] = sizeof(BaseT) == 4 ? kNegInf : kNegInf * 0x10001u;
#pragma unroll
    for (int i = 0; i < kWP; ++i) ep_prev.p[i] = 0u;

    // With three B buffers (16-bit base): the prologue issues B(0) with base
    // chunk 0, then B(1); stage st issues B(st + 2) into buffer (st + 2) % 3 --
    // the one stage st - 1 read, freed by the barrier that starts st -- and, at
    // an even st, chunk st / 2 + 1.  At the start of an even stage the wave
    // waits for everything but B(st + 1) (kEB loads: B(st) and its chunk were
    // issued together at st - 2); at an odd one everything but B(st + 1) and
    // the chunk issued with it.  B is then two stages ahead of its use instead
    // of one.
    issue_all(std::true_type{}, bb[0], 0, qb0, 0);
    if constexpr (kNB == 3) issue_all(std::false_type{}, bb[1], 1, qb1, 0);
    for (int st0 = 0; st0 < nst; st0 += 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int st = st0 + u;
            if (st >= nst) break;
            if constexpr (kNB == 3) {
                if ((u & 1) == 1) tiled::stage_barrier<kEB + kQPieces>();
                else tiled::stage_barrier<kEB>();
            } else {
                if (SPC == 2 && (u & 1) == 1) tiled::stage_barrier<kQPieces>();
                else tiled::stage_barrier<0>();
            }
            BBuf& S = kNB == 3 ? bb[st % 3] : bb[u & 1];
            BBuf& Sn = kNB == 3 ? bb[(st + 2) % 3] : bb[(u + 1) & 1];
            const int cbuf = SPC == 2 ? ((u >> 1) & 1) : (u & 1);
            const QBuf& Q = cbuf ? qb1 : qb0;
            QBuf& Qn = cbuf ? qb0 : qb1;
            const int c_next = st / SPC + 1;
            const bool opens = (st % SPC) == 0;
            if (wave_active) {
                f32x16 acc;
                if (opens) contract(std::true_type{}, S, Q, st, Sn, Qn, c_next, acc, acc_prev, ep_prev, cb_prev, ep_cur);
                else contract(std::false_type{}, S, Q, st, Sn, Qn, c_next, acc, acc_prev, ep_prev, cb_prev, ep_cur);
                acc_prev = acc;
                ep_prev = ep_cur;
                cb_prev = tile_of(st) * kTileCols + 16 * h;
            } else if (opens) {
                issue_all(std::true_type{}, Sn, st + kNB - 1, Qn, c_next);
            } else {
                issue_all(std::false_type{}, Sn, st + kNB - 1, Qn, c_next);
            }
        }
    }
    if (wave_active && nst > 0) {
#pragma unroll
        for (int c = 0; c < kCands; ++c) epi_one(acc_prev, ep_prev, cb_prev, c);
    }
    // no direct-to-LDS load may land after this point: the finish reuses the buffers
    __builtin_amdgcn_s_waitcnt(0x0070 | (0xf << 8));

    // merge the two column halves of the row, one key per row
    const float ov = __shfl_xor(best, 32, 64);
    const int oi = __shfl_xor(bidx, 32, 64);
    if (argmax_better(ov, oi, best, bidx)) {
        best = ov;
        bidx = oi;
    }
    const int m = mw + rl;
    const int fin_m[1] = {(h == 0 && m < a.M) ? m : -1};
    const unsigned long long fin_key[1] = {bidx == INT_MAX ? 0ull : pack_argmax(best, (uint32_t)bidx)};
    tiled_argmax_finish(a, fin_m, fin_key, reinterpret_cast<int*>(&bb[0]));
}

template <int KS8, typename BaseT, typename PriorT>
hipError_t launch_tiled8_inst(const TiledKArgs& ka, int gx, int gy, hipStream_t s) {
    if (ka.V % tiled8::kTileCols == 0)
        hipLaunchKernelGGL((fused_argmax_tiled8_kernel<KS8, BaseT, PriorT, true>), dim3(gx, gy, 1), dim3(tiled8::kThreads),
                           0, s, ka);
    else
        hipLaunchKernelGGL((fused_argmax_tiled8_kernel<KS8, BaseT, PriorT, false>), dim3(gx, gy, 1), dim3(tiled8::kThreads),
                           0, s, ka);
    return hipGetLastError();
}

// Dispatch over r / 128 (2 or 4) and the prior type for one base dtype.
template <typename BaseT>
hipError_t launch_tiled8_for_base(const TiledKArgs& ka, int ks8, int prior_kind, int gx, int gy, hipStream_t s) {
    auto by_prior = [&](auto ks_tag) -> hipError_t {
        constexpr int KS8 = decltype(ks_tag)::value;
        switch (prior_kind) {
            case 0: return launch_tiled8_inst<KS8, BaseT, no_prior_t>(ka, gx, gy, s);
            case 1: return launch_tiled8_inst<KS8, BaseT, float>(ka, gx, gy, s);
            case 2: return launch_tiled8_inst<KS8, BaseT, bf16_t>(ka, gx, gy, s);
            default: return launch_tiled8_inst<KS8, BaseT, f16_t>(ka, gx, gy, s);
        }
    };
    if (ks8 == 2) return by_prior(std::integral_constant<int, 2>{});
    return by_prior(std::integral_constant<int, 4>{});
}

hipError_t launch_tiled8_f32(const TiledKArgs& ka, int ks8, int prior_kind, int gx, int gy, hipStream_t s);
hipError_t launch_tiled8_bf16(const TiledKArgs& ka, int ks8, int prior_kind, int gx, int gy, hipStream_t s);
hipError_t launch_tiled8_f16(const TiledKArgs& ka, int ks8, int prior_kind, int gx, int gy, hipStream_t s);

}  // namespace dels
