/*
 * expert.hpp - expert stage as ONE grouped GEMM launch over all experts.
 *
 * Restates shaders/moe_expert_skip.comp.glsl:25-54 (u = r16(W1 hn + b1),
 * g = r16(GELU-tanh(u)), y = r16(W2 g + b2), out = r16(y + input)) with the
 * pre-LayerNorm added. The reference launches it once per expert over every
 * token and lets unassigned threads return (prism_moe_bench.cpp:280-287);
 * here a workgroup takes one BM-token tile of ONE expert's segment of the
 * router's buckets, so every lane computes.
 *
 * Tile scheduler: the grid is sized for the worst case (ceil(T/BM) + N tiles,
 * rounded up to a multiple of 8). Every wave turns the per-expert counts into
 * a tile prefix sum (a DPP scan), whose total is the number of tiles that
 * exist; workgroup i maps to logical tile (i % 8) * chunk + i / 8, chunk =
 * ceil(total / 8), so that consecutive tiles of one expert land on the same
 * XCD (hardware dispatches workgroups round-robin over the 8 XCDs) and share
 * that XCD's L2 copy of the expert's weights, and every XCD gets an equal
 * share of the tiles; each wave finds its (expert, row block) itself, and
 * workgroups past the tiles do nothing. (The dense FFN stage, no counts:
 * chunk = grid / 8.)
 *
 * Weight streaming: as soon as the tokens are gathered, each wave issues
 * every W1 fragment of its 16*RT output rows (RT*KS 1 KiB fragments, held in
 * registers) right behind the row loads, so W1 arrives while LN2 runs. GEMM1
 * refills the registers of its first KS/2 k-steps with the first half of W2
 * (in flight during GEMM1 and the GELU); GEMM2 issues the second half of W2
 * while it consumes the first. (Issuing all of W2 up front, which the 8-wave
 * variant has the registers for, was measured slower: the rows and W1 then
 * retire behind it.)
 *
 * GEMMs are C^T = W * A^T (weights as the A operand, tokens as columns), so a
 * lane's accumulator holds 4 consecutive channels of one token: 8-byte LDS
 * writes for the GELU tile and for the output tile, which the epilogue adds
 * onto the raw rows kept in LDS for the residual and then scatters back to
 * the tokens' HWC positions as whole 512-byte rows, 16 bytes per lane (fused
 * unpermute; one store instruction covers two rows instead of 16 tokens x
 * 32 bytes).
 *
 * Tile sizes: expert_body (64 tokens, 4 or 8 waves; the weight-streaming
 * scheme above) and expert_body_wide (128 or 96 tokens, 4 waves, d256, for
 * large grids: a weight ring instead of per-pass registers, the residual read
 * again instead of kept in LDS; see its comment). All share the scheduler
 * and give bit-identical results.
 */
#pragma once
#include "common.hpp"

/* Writes the output tile (BM rows of C channels in LDS, row stride STRIDE
 * halfs) to the rows of its tokens: each wave stores BM/NW rows, 16 bytes
 * per lane, so one instruction covers 1 KiB of whole rows instead of 16
 * tokens x 32 bytes. Every LDS read (token ids, then the chunks) is issued
 * before the first store: a read under the store's condition costs one LDS
 * round trip per row pass. */
template <int C, int STRIDE, int BM, int NW, bool NT = false>
__device__ __forceinline__ void expert_store_rows(uint16_t* out, const f16* tile, const int* tok, int wave, int lane) {
    constexpr int CPR = C / 8;    /* 16-byte chunks per row */
    constexpr int RPS = 64 / CPR; /* rows per wave store    */
    constexpr int NI = BM / NW / RPS;
    static_assert(64 % CPR == 0 && (BM / NW) % RPS == 0, "store shape");
    const int c8 = (lane % CPR) * 8;
    int tk[NI];
    h8 v[NI];
#pragma unroll
    for (int it = 0; it < NI; ++it) {
        const int r = wave * (BM / NW) + it * RPS + lane / CPR;
        tk[it] = tok[r];
        v[it] = *reinterpret_cast<const h8*>(tile + r * STRIDE + c8);
    }
#pragma unroll
    for (int it = 0; it < NI; ++it)
        if (tk[it] >= 0) st_row16<NT>(out, ((uint32_t)tk[it] * C + c8) * 2u, v[it]);
}

/* Tile scheduler (see the file comment): every wave finds this workgroup's
 * (expert, first row, row count) itself, or expert -1 past the last tile:
 * the same counts, DPP scan and ballot in each wave, so no LDS broadcast and
 * barrier stand between the counts and the tile's first loads. The results
 * are wave-uniform. */
template <int BM>
__device__ __forceinline__ void expert_schedule(const ExpertArgs& a, int lane, int& e, int& row0, int& rows) {
    if (a.counts) {
        const int c = lane < a.n_experts ? min(a.counts[lane * a.count_stride], a.cap) : 0;
        const int nt = (c + BM - 1) / BM;
        const int incl = wave_incl_scan(nt);
        const int excl = incl - nt;
        /* the tiles that exist (the grid holds the worst case), dealt to the
         * 8 XCDs in equal contiguous chunks: workgroup i runs tile
         * (i % 8) * chunk + i / 8, so no XCD is left with the empty end of
         * the tile range while the others queue a second round */
        const int total = __builtin_amdgcn_readlane(incl, 63);
        const int per_xcd = (total + 7) / 8;
        const int k = blockIdx.x / 8;
        const int L = k < per_xcd ? (blockIdx.x % 8) * per_xcd + k : 0x7fffffff;
        const bool mine = lane < a.n_experts && L >= excl && L < incl;
        const unsigned long long bal = __ballot(mine); /* one lane at most */
        if (bal == 0ull) {
            e = -1;
            row0 = rows = 0;
            return;
        }
        const int o = __builtin_ctzll(bal);
        const int ex = __builtin_amdgcn_readlane(excl, o), co = __builtin_amdgcn_readlane(c, o);
        e = o;
        row0 = (L - ex) * BM;
        rows = min(BM, co - row0);
    } else {
        const int per_xcd = gridDim.x / 8;
        const int L = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
        row0 = L * BM;
        e = row0 < a.n_tokens ? 0 : -1;
        rows = min(BM, a.n_tokens - row0);
    }
}

/* Stages expert e's biases and the tile's token ids (-1 past the segment's
 * end, and for a bucket entry that names no token); rows >= 1. A thread's
 * three loads (b1, b2, its bucket entry; clamped indices, the values past
 * the ends unused) are all issued before its first LDS store, so staging
 * costs one memory round trip. The caller synchronises. */
template <int DIM, int BM, int NT>
__device__ __forceinline__ void expert_stage_tile(const ExpertArgs& a, int e, int row0, int rows, float* s_b1,
                                                  float* s_b2, int* tok) {
    static_assert(DIM <= NT && BM <= NT, "one bias entry and one row a thread");
    const int i = (int)threadIdx.x, ic = min(i, DIM - 1);
    const float b1 = a.b1[(int64_t)e * DIM + ic], b2 = a.b2[(int64_t)e * DIM + ic];
    int t = row0 + i;
    if (a.counts) t = a.perm[(int64_t)e * a.cap + row0 + min(i, rows - 1)]; /* uniform branch */
    if (i >= rows || t < 0 || t >= a.n_tokens) t = -1; /* never follow a stale bucket entry */
    /* the bias stores are unconditional (a thread past the end writes the
       last entry with the value it holds, the same one), so no branch
       invites the compiler to sink their loads next to them */
    s_b1[ic] = b1;
    s_b2[ic] = b2;
    if (i < BM) tok[i] = t;
}

template <int DIM, int BM, int NW, bool WNT = false>
__device__ __forceinline__ void expert_body(const ExpertArgs& a) {
    constexpr int WP = WNT ? 2 : 0; /* weight loads' cache policy */
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    constexpr int NT = 64 * NW;   /* threads                          */
    constexpr int KS = DIM / 32;
    constexpr int LDS = DIM + 8;
    constexpr int TT = BM / 16;   /* token tiles per workgroup        */
    constexpr int RT = DIM / 16 / NW; /* 16-row output tiles per wave */
    constexpr int LPS = DIM / 16; /* LN lanes per row                 */
    constexpr int RPI = 64 / LPS; /* LN rows per wave iteration       */
    static_assert(RT >= 1 && BM % (NW * RPI) == 0, "tile shape");

    __shared__ __attribute__((aligned(16))) f16 xs[BM * LDS]; /* LN2 output, then GELU output */
    __shared__ __attribute__((aligned(16))) f16 hs[BM * LDS]; /* raw rows (residual)          */
    __shared__ float s_b1[DIM], s_b2[DIM];
    __shared__ int tok[BM];

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15;
    const int g = lane >> 4;

    /* ---- schedule ------------------------------------------------------ */
    int e, row0, rows;
    expert_schedule<BM>(a, lane, e, row0, rows);

    if (e >= 0) {
        const FragSrc w1(a.w1 + (int64_t)e * DIM * DIM, DIM * DIM * 2u);
        const FragSrc w2(a.w2 + (int64_t)e * DIM * DIM, DIM * DIM * 2u);
        const int loff = lane * 16;

        expert_stage_tile<DIM, BM, NT>(a, e, row0, rows, s_b1, s_b2, tok);
        __syncthreads();

        /* the gathered rows' loads go out first, then every W1 fragment of
         * this wave's rows, then LN2 runs on the rows while W1 arrives
         * (loads retire in issue order) */
        constexpr int IT = BM / NW / RPI;
        RowChunk rc[IT];
        int rt_tok[IT];
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            rt_tok[it] = tok[wave * (BM / NW) + it * RPI + lane / LPS];
            rc[it] = ln_load<DIM, NW == 8>(a.in, rt_tok[it] >= 0 ? rt_tok[it] : 0); /* none: row 0 */
        }
        h8 wf[RT][KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int r = 0; r < RT; ++r) wf[r][ks] = w1.template load<WP>((wave * RT + r) * KS + ks, loff);
        sched_fence();
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int r = wave * (BM / NW) + it * RPI + lane / LPS;
            ln_store<DIM, false>(rc[it], rt_tok[it] >= 0, xs + r * LDS, hs + r * LDS);
        }
        __syncthreads();

        f4 acc[RT][TT]; /* starts at b1 */
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const int ch = (wave * RT + r) * 16 + 4 * g;
            const f4 bb = {s_b1[ch], s_b1[ch + 1], s_b1[ch + 2], s_b1[ch + 3]};
#pragma unroll
            for (int t = 0; t < TT; ++t) acc[r][t] = bb;
        }
        /* GEMM1: hidden rows [wave*RT*16, +RT*16) for all BM tokens */
        h8 xf[TT], xn[TT]; /* k-step ks+1's operands load during ks's MFMAs */
#pragma unroll
        for (int t = 0; t < TT; ++t) xf[t] = *reinterpret_cast<const h8*>(xs + (16 * t + l16) * LDS + 8 * g);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if (ks + 1 < KS) {
#pragma unroll
                for (int t = 0; t < TT; ++t)
                    xn[t] = *reinterpret_cast<const h8*>(xs + (16 * t + l16) * LDS + 32 * (ks + 1) + 8 * g);
            }
#pragma unroll
            for (int r = 0; r < RT; ++r) {
#pragma unroll
                for (int t = 0; t < TT; ++t) acc[r][t] = mfma_16x16x32(wf[r][ks], xf[t], acc[r][t]);
                if (ks < KS / 2) wf[r][ks] = w2.template load<WP>((wave * RT + r) * KS + ks, loff);
            }
            if (ks + 1 < KS) {
#pragma unroll
                for (int t = 0; t < TT; ++t) xf[t] = xn[t];
            }
            sched_fence();
        }
        __syncthreads(); /* every wave is done reading the LN tile */
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const int ch = (wave * RT + r) * 16 + 4 * g;
            const f4 bb = {s_b2[ch], s_b2[ch + 1], s_b2[ch + 2], s_b2[ch + 3]};
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const h4 u = cvt_h4(acc[r][t]); /* r16(W1 hn + b1) */
                f4 gl;
#pragma unroll
                for (int i = 0; i < 4; ++i) gl[i] = gelu_tanh_h(u[i]);
                *reinterpret_cast<h4*>(xs + (16 * t + l16) * LDS + ch) = cvt_h4(gl);
                acc[r][t] = bb; /* GEMM2 starts at b2 */
            }
        }
        __syncthreads();
        /* GEMM2 */
#pragma unroll
        for (int t = 0; t < TT; ++t) xf[t] = *reinterpret_cast<const h8*>(xs + (16 * t + l16) * LDS + 8 * g);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if (ks + 1 < KS) {
#pragma unroll
                for (int t = 0; t < TT; ++t)
                    xn[t] = *reinterpret_cast<const h8*>(xs + (16 * t + l16) * LDS + 32 * (ks + 1) + 8 * g);
            }
#pragma unroll
            for (int r = 0; r < RT; ++r) {
#pragma unroll
                for (int t = 0; t < TT; ++t) acc[r][t] = mfma_16x16x32(wf[r][ks], xf[t], acc[r][t]);
                /* second half of W2, issued one half ahead of its use */
                if (ks < KS / 2) wf[r][ks + KS / 2] = w2.template load<WP>((wave * RT + r) * KS + ks + KS / 2, loff);
            }
            if (ks + 1 < KS) {
#pragma unroll
                for (int t = 0; t < TT; ++t) xf[t] = xn[t];
            }
            sched_fence();
        }
        /* fused down-projection (last block of the adapted chain): W_dn
         * fragments go out now, while the epilogue below runs */
        constexpr int DO = 128, DRT = DO / 16 / NW;
        static_assert(DRT >= 1, "down-projection shape");
        const bool dn = a.dn_w != nullptr; /* uniform over the launch */
        h8 wd[DRT][KS];
        f4 dbias[DRT];
        if (dn) {
            const FragSrc src_dn(a.dn_w, (unsigned)(DO * DIM * 2));
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int r = 0; r < DRT; ++r) wd[r][ks] = src_dn.load((wave * DRT + r) * KS + ks, loff);
#pragma unroll
            for (int r = 0; r < DRT; ++r) {
                const int ch = (wave * DRT + r) * 16 + 4 * g;
                dbias[r] = f4{a.dn_b[ch], a.dn_b[ch + 1], a.dn_b[ch + 2], a.dn_b[ch + 3]};
            }
        }
        /* epilogue: y = r16(W2 g + b2), out = y + h in fp16 (one rounding),
         * written over the lane's own residual in hs, then whole rows out */
        /* every residual read first, then the adds (read-add-write per
         * element waits one LDS round trip each) */
        h4 hres[TT][RT];
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int r = 0; r < RT; ++r)
                hres[t][r] = *reinterpret_cast<const h4*>(hs + (16 * t + l16) * LDS + (wave * RT + r) * 16 + 4 * g);
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int r = 0; r < RT; ++r)
                *reinterpret_cast<h4*>(hs + (16 * t + l16) * LDS + (wave * RT + r) * 16 + 4 * g) =
                    add_f16x4(cvt_h4(acc[r][t]), hres[t][r]);
        __syncthreads();
        if (!dn) {
            expert_store_rows<DIM, LDS, BM, NW, NW == 8>(a.out, hs, tok, wave, lane);
        } else {
            /* r16(W_dn y + b_dn) (shaders/pw_project_256to128.comp.glsl:25-32,
             * the same arithmetic as prism_project_down_d*) from the output
             * tile in hs into xs (free since GEMM2), then 128-channel rows out */
            f4 dacc[DRT][TT];
#pragma unroll
            for (int r = 0; r < DRT; ++r)
#pragma unroll
                for (int t = 0; t < TT; ++t) dacc[r][t] = dbias[r];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    const h8 yf = *reinterpret_cast<const h8*>(hs + (16 * t + l16) * LDS + 32 * ks + 8 * g);
#pragma unroll
                    for (int r = 0; r < DRT; ++r) dacc[r][t] = mfma_16x16x32(wd[r][ks], yf, dacc[r][t]);
                }
#pragma unroll
            for (int t = 0; t < TT; ++t)
#pragma unroll
                for (int r = 0; r < DRT; ++r)
                    *reinterpret_cast<h4*>(xs + (16 * t + l16) * LDS + (wave * DRT + r) * 16 + 4 * g) =
                        cvt_h4(dacc[r][t]);
            __syncthreads();
            expert_store_rows<DO, LDS, BM, NW, NW == 8>(a.out, xs, tok, wave, lane);
        }
    }

}

/* GELU of one accumulator: u = r16(acc), g = r16(GELU-tanh(u)). */
__device__ __forceinline__ h4 expert_gelu4(const f4& acc) {
    const h4 u = cvt_h4(acc);
    f4 gl;
#pragma unroll
    for (int i = 0; i < 4; ++i) gl[i] = gelu_tanh_h(u[i]);
    return cvt_h4(gl);
}

/* One GEMM of a 128-token tile: acc[r][t] += W(row tile r) * tile^T over the
 * KS k-steps. Weight fragment p = P0 + ks*RT + r of the wave's stream sits in
 * ring[p % PF] and is replaced by fragment p + PF as soon as it has fed its
 * last MFMA. Token tiles go in two halves whose LDS operand reads are double-
 * buffered against each other (half B's reads go out before half A's MFMAs,
 * the next k-step's half A before half B's); every operand fragment feeds RT
 * MFMAs. */
template <int KS, int LDS, int RT, int TT, int PF, int P0, int NF, class Frag>
__device__ __forceinline__ void expert_wide_gemm(f4 (&acc)[RT][TT], h8 (&ring)[PF], const f16* tile, int l16, int g,
                                                 Frag&& frag) {
    constexpr int TH = TT / 2;
    h8 xa[TH], xb[TH];
#pragma unroll
    for (int t = 0; t < TH; ++t) xa[t] = *reinterpret_cast<const h8*>(tile + (16 * t + l16) * LDS + 8 * g);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int t = 0; t < TH; ++t)
            xb[t] = *reinterpret_cast<const h8*>(tile + (16 * (TH + t) + l16) * LDS + 32 * ks + 8 * g);
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int t = 0; t < TH; ++t) acc[r][t] = mfma_16x16x32(ring[(P0 + ks * RT + r) % PF], xa[t], acc[r][t]);
        if (ks + 1 < KS) {
#pragma unroll
            for (int t = 0; t < TH; ++t)
                xa[t] = *reinterpret_cast<const h8*>(tile + (16 * t + l16) * LDS + 32 * (ks + 1) + 8 * g);
        }
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const int p = P0 + ks * RT + r;
#pragma unroll
            for (int t = 0; t < TH; ++t) acc[r][TH + t] = mfma_16x16x32(ring[p % PF], xb[t], acc[r][TH + t]);
            if (p + PF < NF) ring[p % PF] = frag(p + PF);
        }
        sched_fence();
    }
}

/*
 * 128-token tiles on 4 waves (two workgroups per CU), for the large grids of
 * batched launches. Every weight fragment a wave streams feeds 8 token tiles
 * instead of 4, which halves the weight bytes per FLOP through the vector
 * memory pipe, and each token's share of a tile's serial prologue (counts,
 * bucket entries, row gather) halves too, while every LDS operand fragment
 * still feeds 4 MFMAs (one per row tile of the wave). The wave's weights
 * (W1's 64 rows, then W2's) stream through a ring of PF fragments, k-step-
 * major, so W2's first fragments are in flight during the GELU. The LDS holds
 * one BM-row tile (LN2 output, then GELU output, then y) and not the
 * residual: the tile's input rows are read again as GEMM2 ends (by then most
 * have left the XCD's 4 MB L2, so this is a second fetch from the memory
 * side) and added to y as whole rows, 16 bytes per lane. The same body at
 * BM = 96 (6 token tiles) serves large stage calls, whose tile count then
 * leaves less of a last, partly filled round of workgroups.
 * Per output element the arithmetic and its order are those of expert_body
 * (bias in the accumulator, k-steps in order, the same rounding points), so
 * the results are bit-identical to the 64-token kernels.
 * TA = token tiles computed: an expert's last tile is usually partly empty,
 * and in the 128-token kernel one with at most 64 rows runs the TA = 4 body,
 * which gathers, normalises, multiplies, stores and re-reads only those
 * tiles (the empty tiles' results were never stored).
 */
template <int DIM, int BM>
struct ExpertWideLds {
    __attribute__((aligned(16))) f16 xs[BM * (DIM + 8)]; /* LN2 output, GELU output, y */
    float b1[DIM], b2[DIM];
    int tok[BM];
};

template <int DIM, int PF, int BM, int TA>
__device__ __forceinline__ void expert_body_wide(const ExpertArgs& a, ExpertWideLds<DIM, BM>& L, int e, int row0,
                                                 int rows) {
    constexpr int NW = 4;
    constexpr int KS = DIM / 32;
    constexpr int LDS = DIM + 8;
    constexpr int RT = DIM / 16 / NW; /* 16-row output tiles per wave  */
    constexpr int NF = 2 * RT * KS;   /* fragments in the wave's stream */
    constexpr int LPS = DIM / 16;     /* LN lanes per row              */
    constexpr int RPI = 64 / LPS;     /* LN rows per wave iteration    */
    constexpr int IT = BM / NW / RPI;
    static_assert(RT >= 1 && BM % (NW * RPI) == 0 && PF % RT == 0 && PF <= NF, "tile shape");
    static_assert(TA >= 2 && TA % 2 == 0 && 16 * TA <= BM, "active tiles (two equal halves)");
    f16* const xs = L.xs;
    float* const s_b1 = L.b1;
    float* const s_b2 = L.b2;
    int* const tok = L.tok;

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15;
    const int g = lane >> 4;
    /* the waves whose rows all lie past the active tiles skip the row work */
    const bool rw = wave * (BM / NW) < 16 * TA;

    const FragSrc w1(a.w1 + (int64_t)e * DIM * DIM, DIM * DIM * 2u);
    const FragSrc w2(a.w2 + (int64_t)e * DIM * DIM, DIM * DIM * 2u);
    const int loff = lane * 16;
    /* fragment p of the stream: W1 then W2, k-step-major, the wave's RT row tiles */
    auto frag = [&](int p) -> h8 {
        const int q = p % (RT * KS), ks = q / RT, r = q % RT;
        return (p < RT * KS ? w1 : w2).load((wave * RT + r) * KS + ks, loff);
    };
    /* the tile's biases and token ids are staged by the caller */

    /* rows first, then the ring's first fragments; LN2 runs while they arrive */
    RowChunk rc[IT];
    int rt_tok[IT];
    if (rw) {
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            rt_tok[it] = tok[wave * (BM / NW) + it * RPI + lane / LPS];
            rc[it] = ln_load<DIM>(a.in, rt_tok[it] >= 0 ? rt_tok[it] : 0); /* none: row 0 */
        }
    }
    h8 ring[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) ring[p] = frag(p);
    sched_fence();
    if (rw) {
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int r = wave * (BM / NW) + it * RPI + lane / LPS;
            ln_store<DIM, false>(rc[it], rt_tok[it] >= 0, xs + r * LDS, nullptr);
        }
    }
    __syncthreads();

    constexpr int TT = TA; /* token tiles computed */
    f4 acc[RT][TT];
    h4 res[RT][TT];
    /* ---- GEMM1 + GELU ------------------------------------------------- */
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int ch = (wave * RT + r) * 16 + 4 * g;
        const f4 bb = {s_b1[ch], s_b1[ch + 1], s_b1[ch + 2], s_b1[ch + 3]};
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = bb;
    }
    expert_wide_gemm<KS, LDS, RT, TT, PF, 0, NF>(acc, ring, xs, l16, g, frag);
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t) res[r][t] = expert_gelu4(acc[r][t]);
    __syncthreads(); /* every wave is done reading the LN tile */
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t)
            *reinterpret_cast<h4*>(xs + (16 * t + l16) * LDS + (wave * RT + r) * 16 + 4 * g) = res[r][t];
    __syncthreads();
    /* ---- GEMM2 -------------------------------------------------------- */
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int ch = (wave * RT + r) * 16 + 4 * g;
        const f4 bb = {s_b2[ch], s_b2[ch + 1], s_b2[ch + 2], s_b2[ch + 3]};
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = bb;
    }
    expert_wide_gemm<KS, LDS, RT, TT, PF, RT * KS, NF>(acc, ring, xs, l16, g, frag);
    /* the residual rows are fetched a second time now (most have left the
     * XCD's L2 since the gather), so their latency hides behind the y tile's
     * conversion and barriers (issued before GEMM2's last k-step instead, in
     * the registers the weight ring frees there, they measured slower) */
    constexpr int CPR = DIM / 8;  /* 16-byte chunks per row */
    constexpr int RPS = 64 / CPR; /* rows per wave access   */
    constexpr int NI = BM / NW / RPS;
    static_assert(64 % CPR == 0 && (BM / NW) % RPS == 0, "row shape");
    const int c8 = (lane % CPR) * 8;
    h8 hx[NI];
    if (rw) {
#pragma unroll
        for (int it = 0; it < NI; ++it) {
            const int tk = tok[wave * (BM / NW) + it * RPS + lane / CPR];
            hx[it] = ld_row16(a.in, ((uint32_t)(tk >= 0 ? tk : 0) * DIM + c8) * 2u); /* none: row 0, unused */
        }
    }
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t) res[r][t] = cvt_h4(acc[r][t]); /* y = r16(W2 g + b2) */
    __syncthreads(); /* every wave is done reading the GELU tile */
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t)
            *reinterpret_cast<h4*>(xs + (16 * t + l16) * LDS + (wave * RT + r) * 16 + 4 * g) = res[r][t];
    __syncthreads(); /* y tile complete */
    /* ---- out = y + h in fp16 (one rounding), whole rows --------------- */
    if (rw) {
        /* every LDS read first (token ids and y chunks), then the stores: a
           read under the store's condition costs one LDS round trip per row
           pass */
        int tk[NI];
        h8 y[NI];
#pragma unroll
        for (int it = 0; it < NI; ++it) {
            const int r = wave * (BM / NW) + it * RPS + lane / CPR;
            tk[it] = tok[r];
            y[it] = *reinterpret_cast<const h8*>(xs + r * LDS + c8);
        }
#pragma unroll
        for (int it = 0; it < NI; ++it)
            if (tk[it] >= 0) st_row16(a.out, ((uint32_t)tk[it] * DIM + c8) * 2u, add_f16x8(y[it], hx[it]));
    }
}

/* Schedules the tile, then runs the body with every token tile, or (SHORT)
 * with 4 of them when the tile's rows fit there. */
template <int DIM, int PF, int BM, bool SHORT>
__device__ __forceinline__ void expert_wide(const ExpertArgs& a, ExpertWideLds<DIM, BM>& L) {
    static_assert(!SHORT || BM > 64, "the short body is 4 token tiles");
    int e, row0, rows;
    expert_schedule<BM>(a, lane_id(), e, row0, rows);
    if (e < 0) return;
    /* staged once ahead of the body choice (staged inside each body, the
     * compiler merged the two paths' loads and waited for the biases before
     * requesting the bucket entries: two round trips instead of one) */
    expert_stage_tile<DIM, BM, 256>(a, e, row0, rows, L.b1, L.b2, L.tok);
    __syncthreads();
    if (SHORT && rows <= 64) /* uniform */
        expert_body_wide<DIM, PF, BM, 4>(a, L, e, row0, rows);
    else
        expert_body_wide<DIM, PF, BM, BM / 16>(a, L, e, row0, rows);
}

/* 4 waves (2 workgroups per CU) for large grids; 8 waves (each streaming half
 * as many weight rows) when tiles are scarcer than CUs. */
extern "C" __global__ void __launch_bounds__(256, 2) prism_expert_d256_bm64(ExpertArgs a) {
    expert_body<256, 64, 4>(a);
}
extern "C" __global__ void __launch_bounds__(256, 2) prism_expert_d128_bm64(ExpertArgs a) {
    expert_body<128, 64, 4>(a);
}
extern "C" __global__ void __launch_bounds__(512, 1) prism_expert_d256_bm64_w8(ExpertArgs a) {
    if (a.wnt) /* uniform */
        expert_body<256, 64, 8, true>(a);
    else
        expert_body<256, 64, 8>(a);
}
extern "C" __global__ void __launch_bounds__(512, 1) prism_expert_d128_bm64_w8(ExpertArgs a) {
    expert_body<128, 64, 8>(a);
}
/* 128-token tiles, 4 waves, 2 workgroups per CU: the large grids of batched
 * launches (no fused down-projection) */
extern "C" __global__ void __launch_bounds__(256, 2) prism_expert_d256_bm128(ExpertArgs a) {
    __shared__ ExpertWideLds<256, 128> lds;
    expert_wide<256, 12, 128, true>(a, lds);
}
/* 96-token tiles of the same body: a large stage call's tile count then
 * rounds up to whole rounds of the CUs' workgroup slots with less idle tail */
extern "C" __global__ void __launch_bounds__(256, 2) prism_expert_d256_bm96(ExpertArgs a) {
    __shared__ ExpertWideLds<256, 96> lds;
    expert_wide<256, 12, 96, false>(a, lds); /* the short body measured slower here */
}
