/*
 * attn.hpp - attention stage: one workgroup per 8x8 window, 4 waves.
 *
 * Restates shaders/split2_qkv_attn_d256.comp.glsl:24-79 (window mapping
 * :25-33, zero-vector padded slots :31-37, QKV :39-51, softmax core :53-69,
 * out-proj + fp16 residual :71-78) with the pre-LayerNorm added, as:
 *
 *  1. LN1 of the window's 64 slots -> xs (LDS, fp16), the raw rows -> os
 *     (they are the residual; the out-proj's epilogue reads them from there,
 *     so x is fetched from HBM once). Padded slots are zero, so their keys
 *     and values are the bias (with LN1's affine folded into W_qkv and the
 *     bias, a block with beta != 0 gives padded windows the PAD body, which
 *     restores the blob's own bias there). With a fused
 *     up-projection (the adapted chain's first block) the input rows have 128
 *     channels and x = r16(ReLU(W_up e + b_up)) is computed into os first
 *     (shaders/pw_project_128to256.comp.glsl:25-37, as project.hpp).
 *  2. Wave w owns heads w and w+4 (8-wave variant: head w). Per head, one
 *     MFMA GEMM pass over the model dim produces Q^T and K^T (rows = channel,
 *     cols = token) and V
 *     (rows = token, cols = channel), fp32 accumulate, bias, fp16 round.
 *  3. S^T = K Q^T is one MFMA per 16x16 tile straight from those registers:
 *     an accumulator lane holds 4 consecutive channels of one token, which is
 *     exactly a k-slice of an operand under the permuted k numbering
 *     k(g, j) = 16*(j/4) + 4g + j%4. Softmax runs down the key axis: 16
 *     values in-lane plus two cross-lane xor shuffles. P = exp(...) stays in
 *     registers and O^T = V^T P^T is again register-to-register MFMA.
 *     O^T is normalised, rounded to fp16 and kept in registers until every
 *     wave has finished reading xs; then all heads' O^T go to xs.
 *  4. Out-proj C^T = Wo * O^T, bias, fp16 round, + x from os (fp16 round),
 *     written over the lane's residual in os; the finished tile leaves as
 *     whole 512-byte rows (16 bytes per lane) after the router GEMM (4 waves)
 *     or at the very end (8 waves).
 *  5. Routed variants (NPT > 0, the block chain's MoE blocks) route that
 *     output tile from os: waves 0-3 each take 16 tokens through
 *     LN2 + router GEMM + argmax (route_token, whose W_r fragments continue
 *     the weight ring), then the window's counting sort (LDS histogram, one
 *     global atomic per present expert, bucket scatter). This replaces the
 *     router launch and its re-read of h.
 *
 * Windows whose slots 32-63 are all padded (a grid's bottom window row with
 * 4 or fewer rows) take a body that computes only token tiles 0 and 1 (HALF,
 * below): the other tiles' keys and values are the bias alone.
 *
 * Weight streaming: every wave reads one fixed sequence of 1 KiB weight
 * fragments (head A's QKV k-steps, head B's, the out-proj's, the router's) through a
 * register ring PF fragments deep, so loads run 2 k-steps ahead of the MFMAs
 * and the next head's and the out-proj's first fragments are in flight while
 * the softmax math runs. All workgroups read the same 0.5 MiB per block,
 * which stays L2-resident. Biases are staged in LDS once; the LayerNorms'
 * affines are folded into W_qkv and W_r on the host.
 */
#pragma once
#include "route.hpp"

template <int DIM, int HD, int NW, int NPT>
struct AttnShape {
    static constexpr int KS = DIM / 32;            /* k-steps over the model dim     */
    static constexpr int CT = HD / 16;             /* 16-channel tiles per head      */
    static constexpr int FPK = 3 * CT;             /* QKV fragments per k-step       */
    static constexpr int HEADF = KS * FPK;         /* fragments per head             */
    static constexpr int HPW = 8 / NW;             /* heads per wave                 */
    static constexpr int ORT = DIM / 16 / NW;      /* out-proj row tiles per wave    */
    static constexpr int OUTF = KS * ORT;          /* out-proj fragments             */
    static constexpr int RBASE = HPW * HEADF + OUTF; /* sequence length, no routing  */
    /* 8 waves, even NPT: waves w and w+4 route the same 16 tokens, each over
     * half of the expert row tiles (RPT of them) */
    static constexpr bool RSPLIT = NW == 8 && NPT > 0 && NPT % 2 == 0;
    static constexpr int RPT = RSPLIT ? NPT / 2 : NPT;
    static constexpr int TOTAL = RBASE + RPT * KS;   /* routing waves add W_r        */
    static constexpr int PF = 2 * FPK;             /* ring depth (2 k-steps ahead)   */
    static constexpr int LDS = DIM + 8;            /* padded LDS row, halfs          */
};

/* Fragment p of wave `wave`'s sequence: head A's QKV k-steps, head B's, the
 * out-proj's, then (routing waves) the router's, k-step-major (p is a
 * compile-time constant or depends only on the head index, so every branch
 * is wave-uniform). */
template <int DIM, int HD, int NW, int NPT>
__device__ __forceinline__ h8 attn_frag(const FragSrc& wqkv, const FragSrc& wo, const FragSrc& wr, int wave, int p,
                                        int loff) {
    using S = AttnShape<DIM, HD, NW, NPT>;
    if (p < S::HPW * S::HEADF) {
        const int hh = p / S::HEADF, q = p % S::HEADF;
        const int ks = q / S::FPK, f = q % S::FPK;
        const int mat = f / S::CT, c = f % S::CT; /* 0 = Q, 1 = K, 2 = V */
        const int h = wave + NW * hh;
        const int rt = (mat * DIM + h * HD) / 16 + c;
        return wqkv.load(rt * S::KS + ks, loff);
    }
    if (NPT == 0 || p < S::RBASE) {
        const int q = p - S::HPW * S::HEADF;
        const int ks = q / S::ORT, r = q % S::ORT;
        return wo.load((wave * S::ORT + r) * S::KS + ks, loff);
    }
    const int q = p - S::RBASE;
    constexpr int R = S::RPT > 0 ? S::RPT : 1;
    const int rt0 = S::RSPLIT && wave >= 4 ? S::RPT : 0; /* the upper half's row tiles */
    return wr.load((rt0 + q % R) * S::KS + q / R, loff);
}

/* The workgroup's LDS, declared once per kernel: both instantiations of the
 * body (windows with and without padded slots) use the same arrays. */
template <int DIM, int NPT>
struct AttnLds {
    __attribute__((aligned(16))) f16 xs[64 * (DIM + 8)];
    __attribute__((aligned(16))) f16 os[64 * (DIM + 8)];
    float bqkv[3 * DIM];
    float bqkv_pad[3 * DIM]; /* PAD bodies only */
    float bo[DIM];
    float br[NPT > 0 ? 16 * NPT : 1]; /* router bias */
};

/* PAD: the window has padded slots and the block's LN1 beta is not zero, so
 * those slots' keys and values need the unfolded bias (a separate
 * instantiation keeps that code, and its branches, out of every other
 * window's instruction schedule). vmask bit s: slot s holds a token.
 * HALF: slots 32-63 are all padded (the bottom windows of a grid whose
 * height leaves 4 or fewer rows in the last window row, e.g. 68 rows), so
 * token tiles 2 and 3 are never queries, never stored and never routed: only
 * their keys and values are used, and those are the bias alone (the zero LN1
 * output adds nothing to the accumulator that starts at the bias; with PAD,
 * the fix-up below sets them). The body then computes Q, the softmax rows,
 * O, the out-projection, LN1 (and the fused up-projection) and the routing
 * for tiles 0 and 1 only; every stored value is computed as in the full
 * body. */
template <int DIM, int HD, int NW, int NPT, bool PAD, bool HALF = false, bool FFN = false>
__device__ __forceinline__ void attn_window_body(const AttnArgs& a, AttnLds<DIM, NPT>& L,
                                                 unsigned long long vmask) {
    constexpr int TQ = HALF ? 2 : 4; /* token tiles that hold tokens */
    static_assert(DIM / HD == 8, "8 heads");
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    static_assert(NPT >= 0 && NPT <= 4, "up to 64 experts");
    using S = AttnShape<DIM, HD, NW, NPT>;
    constexpr int NT = 64 * NW;         /* threads                         */
    constexpr int KS = S::KS, CT = S::CT, LDS = S::LDS, ORT = S::ORT;
    /* ring depth: 2 k-steps ahead; 1 in the rare PAD body, whose padded-slot
     * fix-up needs the registers; 4 in the HALF body, whose k-steps have half
     * the MFMAs to cover an L2 round trip with (and which has half the
     * accumulators) */
    constexpr int PF = PAD ? (HALF ? 2 * S::FPK : S::FPK) : (HALF ? 4 * S::FPK : S::PF);
    constexpr float LOG2E = 1.4426950408889634f;
    const float scale = (HD == 32) ? 0.1767766953f : 1.0f / sqrtf((float)HD);
    const float sl2 = scale * LOG2E;

    static_assert(LDS == DIM + 8, "LDS row");
    f16* const xs = L.xs;
    f16* const os = L.os;
    float* const s_bqkv = L.bqkv;
    float* const s_bqkv_pad = L.bqkv_pad;
    float* const s_bo = L.bo;
    float* const s_br = L.br;
    /* routing scratch aliases the QKV biases, dead after the barrier ahead of
     * the out-proj */
    static_assert(3 * DIM >= 5 * 64, "routing scratch fits the QKV bias area");
    int* const r_hist = reinterpret_cast<int*>(s_bqkv) + 64; /* [64] window histogram */
    int* const r_base = r_hist + 64;                     /* [64] bucket bases        */
    int* const r_e = r_base + 64;                        /* [64] expert per slot     */
    int* const r_rank = r_e + 64;                        /* [64] rank in its bucket  */

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15;
    const int g = lane >> 4;

    const int wg = blockIdx.x;
    const int frame = wg / a.windows_per_frame;
    const int wi = wg - frame * a.windows_per_frame;
    const int wy = wi / a.wx;
    const int wxx = wi - wy * a.wx;
    const uint16_t* in = a.in + (int64_t)frame * a.in_frame_elems;
    uint16_t* out = a.out + (int64_t)frame * a.frame_elems;

    const FragSrc src_qkv(a.wqkv, 3u * DIM * DIM * 2u);
    const FragSrc src_o(a.wo, 1u * DIM * DIM * 2u);
    const FragSrc src_r(NPT > 0 ? a.wr : a.wo, NPT > 0 ? 16u * NPT * DIM * 2u : 0u);
    const int loff = lane * 16;
    /* waves 0-3 route tiles 0-3 of the window (waves w and w+4 tile w % 4
     * when split). Every wave's ring runs into W_r's first fragments (the
     * refills are unconditional: a refill under a wave-dependent branch makes
     * the compiler's load counting at the join wait for the refills just
     * issued, a full L2 round trip per k-step at the end of the
     * out-projection); only the routing waves consume them. */
    const bool routes = NPT > 0 && (S::RSPLIT ? (wave & 3) < TQ : wave < TQ);

    /* ---- 1. LN1 --------------------------------------------------------
     * The window's rows (HBM) are requested first, then the weight ring and
     * the parameters (L2). Loads complete in issue order, so the first wait
     * for a parameter also covers the rows: one memory round trip before
     * the math, not two. */
    constexpr int LPS = DIM / 16;
    constexpr int SPI = 64 / LPS;       /* slots per wave iteration */
    constexpr int SPW = 64 / NW;        /* slots per wave           */
    constexpr int IT = SPW / SPI;
    /* fused up-projection: the window's 128-channel input rows (16 chunks
     * of 16 bytes each, EPT per thread) and this wave's W_up fragments */
    constexpr int UIN = 128, UKS = UIN / 32, UPR = DIM / 16 / NW, EPT = 64 * (UIN / 8) / NT;
    static_assert(UPR >= 1 && EPT >= 1, "up-projection shape");
    const bool up = a.up_w != nullptr; /* uniform over the launch */
    /* HALF: the waves whose slots are all padded skip LN1 (their rows of xs
     * and os are never read) */
    const bool lnw = !HALF || wave * SPW < 16 * TQ;
    RowChunk rc[IT];
    bool valid[IT];
    h8 erow[EPT];
    h8 wup[UPR][UKS];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int s = wave * SPW + it * SPI + lane / LPS;
        const int gy = wy * 8 + (s >> 3), gx = wxx * 8 + (s & 7);
        valid[it] = gy < a.H && gx < a.W;
    }
    if (!up) {
        if (lnw) {
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const int s = wave * SPW + it * SPI + lane / LPS;
                const int gy = wy * 8 + (s >> 3), gx = wxx * 8 + (s & 7);
                rc[it] = ln_load<DIM, NW == 8>(in, valid[it] ? gy * a.W + gx : wy * 8 * a.W + wxx * 8); /* padded: slot 0's row */
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            const int q = threadIdx.x + k * NT, sl = q / (UIN / 8), c8 = (q % (UIN / 8)) * 8;
            const int gy = wy * 8 + (sl >> 3), gx = wxx * 8 + (sl & 7);
            const bool ok = gy < a.H && gx < a.W;
            /* a padded slot reads slot 0's row (in the map) and takes zeros:
               no branch around the load, so all of them go out together */
            const int pix = ok ? gy * a.W + gx : wy * 8 * a.W + wxx * 8;
            const h8 v = *reinterpret_cast<const h8*>(in + (int64_t)pix * UIN + c8);
            erow[k] = ok ? v : h8{};
        }
        const FragSrc src_up(a.up_w, (unsigned)(DIM * UIN * 2));
#pragma unroll
        for (int ks = 0; ks < UKS; ++ks)
#pragma unroll
            for (int r = 0; r < UPR; ++r) wup[r][ks] = src_up.load((wave * UPR + r) * UKS + ks, lane * 16);
    }
    sched_fence();

    /* weight ring: the first PF fragments */
    h8 ring[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) ring[p] = attn_frag<DIM, HD, NW, NPT>(src_qkv, src_o, src_r, wave, p, loff);
    sched_fence();

    /* block chain: clear the next block's counters (its previous reader, that
     * block's expert stage of the previous chain, has finished) */
    if (NPT > 0 && a.zero_next && blockIdx.x == 0 && threadIdx.x < a.n_experts)
        a.zero_next[threadIdx.x * a.count_stride] = 0;
    /* every parameter is staged here, before LN1. All of a thread's
     * parameter loads are issued before its first LDS store (a loop of
     * load-then-store passes waits one L2 round trip per pass); loads retire
     * in issue order, so the stores wait for the rows, the ring's first
     * fragments and these loads together: one memory round trip, which LN1
     * and the QKV GEMM wait for anyway. The barrier after LN1 publishes them
     * (each wave starts its LN1 as soon as its own rows are in, without
     * waiting for the other waves' stores) */
    {
        constexpr int NQ = (3 * DIM + NT - 1) / NT, NB = (DIM + NT - 1) / NT;
        constexpr int NR = NPT > 0 ? (16 * NPT + NT - 1) / NT : 0, NRA = NR > 0 ? NR : 1;
        const int tid = (int)threadIdx.x;
        float pq[NQ], pp[NQ], pb[NB], pr[NRA];
#pragma unroll
        for (int k = 0; k < NQ; ++k) pq[k] = a.bqkv[min(tid + k * NT, 3 * DIM - 1)];
        if constexpr (PAD) {
#pragma unroll
            for (int k = 0; k < NQ; ++k) pp[k] = a.bqkv_pad[min(tid + k * NT, 3 * DIM - 1)];
        }
#pragma unroll
        for (int k = 0; k < NB; ++k) pb[k] = a.bo[min(tid + k * NT, DIM - 1)];
#pragma unroll
        for (int k = 0; k < NR; ++k) pr[k] = a.br[min(tid + k * NT, 16 * NPT - 1)];
        /* the stores are unconditional: a thread past an array's end writes
           its last entry with the value it holds (the same value), so no
           branch invites the compiler to sink a load next to its store */
#pragma unroll
        for (int k = 0; k < NQ; ++k) {
            s_bqkv[min(tid + k * NT, 3 * DIM - 1)] = pq[k];
            if constexpr (PAD) s_bqkv_pad[min(tid + k * NT, 3 * DIM - 1)] = pp[k];
        }
#pragma unroll
        for (int k = 0; k < NB; ++k) s_bo[min(tid + k * NT, DIM - 1)] = pb[k];
#pragma unroll
        for (int k = 0; k < NR; ++k) s_br[min(tid + k * NT, 16 * NPT - 1)] = pr[k];
    }
    if (!up) {
        if (lnw) {
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const int row = (wave * SPW + it * SPI + lane / LPS) * LDS;
                ln_store<DIM>(rc[it], valid[it], xs + row, os + row); /* os: the raw rows (residual) */
            }
        }
    } else {
        /* x = r16(ReLU(W_up e + b_up)) for the window's slots, the same
         * arithmetic as prism_project_up_d* (bias in the accumulator, k-steps
         * in order), into os as the raw rows; padded slots are zero. The 128-
         * channel rows are staged in xs first (B operands). */
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            const int q = threadIdx.x + k * NT, sl = q / (UIN / 8), c8 = (q % (UIN / 8)) * 8;
            *reinterpret_cast<h8*>(xs + sl * LDS + c8) = erow[k];
        }
        __syncthreads();
        f4 uacc[UPR][4];
#pragma unroll
        for (int r = 0; r < UPR; ++r) {
            const int ch = (wave * UPR + r) * 16 + 4 * g;
            const f4 bb = {a.up_b[ch], a.up_b[ch + 1], a.up_b[ch + 2], a.up_b[ch + 3]};
#pragma unroll
            for (int t = 0; t < 4; ++t) uacc[r][t] = bb;
        }
#pragma unroll
        for (int ks = 0; ks < UKS; ++ks)
#pragma unroll
            for (int t = 0; t < TQ; ++t) {
                const h8 xf = *reinterpret_cast<const h8*>(xs + (16 * t + l16) * LDS + 32 * ks + 8 * g);
#pragma unroll
                for (int r = 0; r < UPR; ++r) uacc[r][t] = mfma_16x16x32(wup[r][ks], xf, uacc[r][t]);
            }
#pragma unroll
        for (int t = 0; t < TQ; ++t) {
            const int sl = 16 * t + l16;
            const bool ok = wy * 8 + (sl >> 3) < a.H && wxx * 8 + (sl & 7) < a.W;
#pragma unroll
            for (int r = 0; r < UPR; ++r) {
                f4 v = uacc[r][t];
                /* max(r16(v), 0) == r16(max(v, 0)): fp16 rounding is monotonic */
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = fmaxf(v[i], 0.f);
                const h4 x4 = cvt_h4(v);
                *reinterpret_cast<h4*>(os + sl * LDS + (wave * UPR + r) * 16 + 4 * g) = ok ? x4 : h4{};
            }
        }
        __syncthreads(); /* x complete in os; the staging in xs is dead */
        if (lnw) {
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const int row = (wave * SPW + it * SPI + lane / LPS) * LDS;
                const int ca = (lane % LPS) * 8;
                const RowChunk xr{*reinterpret_cast<const h8*>(os + row + ca),
                                  *reinterpret_cast<const h8*>(os + row + ca + DIM / 2)};
                ln_store<DIM>(xr, valid[it], xs + row, nullptr);
            }
        }
    }
    __syncthreads();

    /* ---- 2./3. per head ----------------------------------------------- */
    static_assert(S::HEADF % PF == 0, "ring slots must not depend on the head index");
    h4 okeep[S::HPW][CT][4]; /* O^T of each head (channel tile, query tile) until xs is free */
#pragma unroll
    for (int hh = 0; hh < S::HPW; ++hh) {
        /* keeps the head-invariant xs reads inside the loop (hoisting all of
         * them out would pin 32 fragments in registers) */
        asm volatile("" ::: "memory");
        const int h = wave + NW * hh;
        /* accumulators start at the bias, so the MFMAs add it.
         * Q^T/K^T element i: channel 16c+4g+i, token 16t+l16.
         * V element i: token 16t+4g+i, channel 16c+l16. */
        f4 accQ[CT][4], accK[CT][4], accV[4][CT];
#pragma unroll
        for (int c = 0; c < CT; ++c) {
            const int chq = h * HD + 16 * c + 4 * g;
            const f4 bq = {s_bqkv[chq], s_bqkv[chq + 1], s_bqkv[chq + 2], s_bqkv[chq + 3]};
            const f4 bk = {s_bqkv[DIM + chq], s_bqkv[DIM + chq + 1], s_bqkv[DIM + chq + 2], s_bqkv[DIM + chq + 3]};
            const float bv = s_bqkv[2 * DIM + h * HD + 16 * c + l16];
#pragma unroll
            for (int t = 0; t < 4; ++t) { accQ[c][t] = bq; accK[c][t] = bk; accV[t][c] = f4{bv, bv, bv, bv}; }
        }

        /* B operands double-buffered: k-step ks+1's LDS reads go out before
         * k-step ks's MFMAs, so their latency hides behind them */
        h8 xf[4], xn[4];
#pragma unroll
        for (int t = 0; t < TQ; ++t) xf[t] = *reinterpret_cast<const h8*>(xs + (16 * t + l16) * LDS + 8 * g);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if (ks + 1 < KS) {
#pragma unroll
                for (int t = 0; t < TQ; ++t)
                    xn[t] = *reinterpret_cast<const h8*>(xs + (16 * t + l16) * LDS + 32 * (ks + 1) + 8 * g);
            }
#pragma unroll
            for (int f = 0; f < S::FPK; ++f) {
                const int p = hh * S::HEADF + ks * S::FPK + f;
                const h8 w = ring[p % PF];
                const int mat = f / CT, c = f % CT;
#pragma unroll
                for (int t = 0; t < TQ; ++t) {
                    if (mat == 0) accQ[c][t] = mfma_16x16x32(w, xf[t], accQ[c][t]);
                    else if (mat == 1) accK[c][t] = mfma_16x16x32(w, xf[t], accK[c][t]);
                    else accV[t][c] = mfma_16x16x32(xf[t], w, accV[t][c]);
                }
                if (p + PF < S::TOTAL)
                    ring[p % PF] = attn_frag<DIM, HD, NW, NPT>(src_qkv, src_o, src_r, wave, p + PF, loff);
            }
            if (ks + 1 < KS) {
#pragma unroll
                for (int t = 0; t < TQ; ++t) xf[t] = xn[t];
            }
            sched_fence();
        }

        /* fp16 round (the bias is already in) */
        h4 q4[CT][4], k4[CT][4], v4[4][CT];
#pragma unroll
        for (int c = 0; c < CT; ++c)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                q4[c][t] = cvt_h4(accQ[c][t]);
                k4[c][t] = cvt_h4(accK[c][t]);
                v4[t][c] = cvt_h4(accV[t][c]);
            }

        /* A padded slot's input is the zero vector, so its key and value are
         * r16 of the bias alone, without the LN1 beta term (W beta) that
         * bqkv carries for the window's tokens. (Its query and output are
         * never used.) */
        if constexpr (PAD) {
#pragma unroll
            for (int c = 0; c < CT; ++c) {
                const int chk = DIM + h * HD + 16 * c + 4 * g;
                const h4 bk = cvt_h4(f4{s_bqkv_pad[chk], s_bqkv_pad[chk + 1], s_bqkv_pad[chk + 2],
                                        s_bqkv_pad[chk + 3]});
                const f16 bv = (f16)s_bqkv_pad[2 * DIM + h * HD + 16 * c + l16];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    /* slots 16t..16t+15 (uniform): all present, all padded
                     * (a bottom-edge window's last rows), or mixed */
                    const unsigned tm = (unsigned)(vmask >> (16 * t)) & 0xffffu;
                    if (t >= TQ || tm == 0u) {
                        k4[c][t] = bk;
                        v4[t][c] = h4{bv, bv, bv, bv};
                    } else if (tm != 0xffffu) {
                        if (!((tm >> l16) & 1u)) k4[c][t] = bk;
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (!((tm >> (4 * g + i)) & 1u)) v4[t][c][i] = bv;
                    }
                }
            }
        }

        /* Per query tile qt: S^T[kt] (element i = key 16kt+4g+i, query 16qt+l16),
         * softmax down the key axis (16 values in-lane, then the 4 lane groups),
         * P kept as fp16 operands for the P.V MFMA. */
        h4 p[4][4];
        float inv[4];
#pragma unroll
        for (int qt = 0; qt < TQ; ++qt) {
            f4 s[4];
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                if constexpr (CT == 2) {
                    const h8 ka = {k4[0][kt][0], k4[0][kt][1], k4[0][kt][2], k4[0][kt][3],
                                   k4[1][kt][0], k4[1][kt][1], k4[1][kt][2], k4[1][kt][3]};
                    const h8 qb = {q4[0][qt][0], q4[0][qt][1], q4[0][qt][2], q4[0][qt][3],
                                   q4[1][qt][0], q4[1][qt][1], q4[1][qt][2], q4[1][qt][3]};
                    s[kt] = mfma_16x16x32(ka, qb, f4_zero());
                } else {
                    s[kt] = mfma_16x16x16(k4[0][kt], q4[0][qt], f4_zero());
                }
            }
            const float m = max_groups(max16(s));
            /* exp(scale * (s - m)) = 2^(s * sl2 - m * sl2) */
            const float msl = m * sl2;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                f4 e;
#pragma unroll
                for (int i = 0; i < 4; ++i) e[i] = fast_exp2(__builtin_fmaf(s[kt][i], sl2, -msl));
                p[kt][qt] = cvt_h4(e);
            }
        }
        /* The softmax denominators on the matrix cores: an all-ones A operand
         * against P^T sums each query's 64 fp16 weights (the P that the P.V
         * MFMAs use) into every lane of its column. */
        {
            const h8 ones = {(f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f};
#pragma unroll
            for (int qt = 0; qt < TQ; ++qt) {
                f4 z = f4_zero();
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const h8 pb = {p[2 * st][qt][0], p[2 * st][qt][1], p[2 * st][qt][2], p[2 * st][qt][3],
                                   p[2 * st + 1][qt][0], p[2 * st + 1][qt][1], p[2 * st + 1][qt][2],
                                   p[2 * st + 1][qt][3]};
                    z = mfma_16x16x32(ones, pb, z);
                }
                inv[qt] = fast_rcp(vmax(z[0], 1e-6f));
            }
        }

        /* O^T[channel tile dt][query tile qt] = V^T P^T over 64 keys (2 k-steps) */
#pragma unroll
        for (int dt = 0; dt < CT; ++dt)
#pragma unroll
            for (int qt = 0; qt < TQ; ++qt) {
                f4 o = f4_zero();
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const h8 va = {v4[2 * st][dt][0], v4[2 * st][dt][1], v4[2 * st][dt][2], v4[2 * st][dt][3],
                                   v4[2 * st + 1][dt][0], v4[2 * st + 1][dt][1], v4[2 * st + 1][dt][2],
                                   v4[2 * st + 1][dt][3]};
                    const h8 pb = {p[2 * st][qt][0], p[2 * st][qt][1], p[2 * st][qt][2], p[2 * st][qt][3],
                                   p[2 * st + 1][qt][0], p[2 * st + 1][qt][1], p[2 * st + 1][qt][2],
                                   p[2 * st + 1][qt][3]};
                    o = mfma_16x16x32(va, pb, o);
                }
                okeep[hh][dt][qt] = cvt_h4(o * inv[qt]);
            }
    }

    /* every wave has read xs for the last time: O of all heads goes there */
    __syncthreads();
#pragma unroll
    for (int hh = 0; hh < S::HPW; ++hh)
#pragma unroll
        for (int dt = 0; dt < CT; ++dt)
#pragma unroll
            for (int qt = 0; qt < TQ; ++qt)
                *reinterpret_cast<h4*>(xs + (16 * qt + l16) * LDS + (wave + NW * hh) * HD + 16 * dt + 4 * g) =
                    okeep[hh][dt][qt];
    if constexpr (NPT > 0) /* the QKV biases are dead now */
        if (threadIdx.x < 64) r_hist[threadIdx.x] = 0;
    __syncthreads();

    /* ---- 4. out-proj + residual --------------------------------------- */
    f4 acc[ORT][4]; /* starts at the out-proj bias */
#pragma unroll
    for (int r = 0; r < ORT; ++r) {
        const int ch = (wave * ORT + r) * 16 + 4 * g;
        const f4 bo = {s_bo[ch], s_bo[ch + 1], s_bo[ch + 2], s_bo[ch + 3]};
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[r][t] = bo;
    }
    h8 of[4], on[4]; /* double-buffered like the QKV operands */
#pragma unroll
    for (int t = 0; t < TQ; ++t) of[t] = *reinterpret_cast<const h8*>(xs + (16 * t + l16) * LDS + 8 * g);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        if (ks + 1 < KS) {
#pragma unroll
            for (int t = 0; t < TQ; ++t)
                on[t] = *reinterpret_cast<const h8*>(xs + (16 * t + l16) * LDS + 32 * (ks + 1) + 8 * g);
        }
#pragma unroll
        for (int r = 0; r < ORT; ++r) {
            const int p = S::HPW * S::HEADF + ks * ORT + r;
            const h8 w = ring[p % PF];
#pragma unroll
            for (int t = 0; t < TQ; ++t) acc[r][t] = mfma_16x16x32(w, of[t], acc[r][t]);
            if (p + PF < S::TOTAL)
                ring[p % PF] = attn_frag<DIM, HD, NW, NPT>(src_qkv, src_o, src_r, wave, p + PF, loff);
        }
        if (ks + 1 < KS) {
#pragma unroll
            for (int t = 0; t < TQ; ++t) of[t] = on[t];
        }
        sched_fence();
    }
    /* po = r16(Wo a + bo); y = po + x in fp16 (one rounding), over the
     * residual: the tile leaves the CU as whole rows (below). All of this
     * lane's residual reads go out before the first add (read-add-write per
     * element waits one LDS round trip each) */
    h4 xres[4][ORT];
#pragma unroll
    for (int t = 0; t < TQ; ++t)
#pragma unroll
        for (int r = 0; r < ORT; ++r)
            xres[t][r] = *reinterpret_cast<const h4*>(os + (16 * t + l16) * LDS + (wave * ORT + r) * 16 + 4 * g);
#pragma unroll
    for (int t = 0; t < TQ; ++t)
#pragma unroll
        for (int r = 0; r < ORT; ++r)
            *reinterpret_cast<h4*>(os + (16 * t + l16) * LDS + (wave * ORT + r) * 16 + 4 * g) =
                add_f16x4(cvt_h4(acc[r][t]), xres[t][r]);
    __syncthreads(); /* y tile complete in os */
    /* ---- 6. y rows out, 16 bytes per lane (a wave store covers whole rows).
     * Loads and stores retire through one counter (vmcnt), so a load or a
     * returning atomic issued after them waits for them too. The 4-wave
     * kernel (large grids) issues them once the router GEMM's loads are all
     * out, so they drain during the counting sort; the 8-wave kernel (small
     * grids, where that sort's device atomics are the critical path) last. */
    auto store_rows = [&]() {
        constexpr int CPR = DIM / 8;  /* 16-byte chunks per row */
        constexpr int RPS = 64 / CPR; /* rows per wave store    */
        constexpr int NI = SPW / RPS;
        static_assert(64 % CPR == 0 && SPW % RPS == 0, "row store shape");
        const int c8 = (lane % CPR) * 8;
        /* every LDS read first, then the stores (a read under the store's
           condition costs one LDS round trip per row pass) */
        h8 v[NI];
#pragma unroll
        for (int it = 0; it < NI; ++it)
            v[it] = *reinterpret_cast<const h8*>(os + (wave * SPW + it * RPS + lane / CPR) * LDS + c8);
#pragma unroll
        for (int it = 0; it < NI; ++it) {
            const int sl = wave * SPW + it * RPS + lane / CPR;
            const int gy = wy * 8 + (sl >> 3), gx = wxx * 8 + (sl & 7);
            if (gy < a.H && gx < a.W)
                st_row16<NW == 8>(out, ((uint32_t)(gy * a.W + gx) * DIM + c8) * 2u, v[it]);
        }
    };

    /* ---- 5. fused routing (moe_router.comp.glsl:24-52 + counting sort) -- */
    if constexpr (NPT > 0) {
        auto rfrag = [&](int rt, int ks) {
            const int p = S::RBASE + ks * S::RPT + rt;
            const h8 w = ring[p % PF];
            if (p + PF < S::TOTAL)
                ring[p % PF] = attn_frag<DIM, HD, NW, NPT>(src_qkv, src_o, src_r, wave, p + PF, loff);
            return w;
        };
        if constexpr (S::RSPLIT) {
            /* waves w and w+4: tokens 16(w%4)..+15, expert row tiles [0, RPT) and
             * [RPT, NPT); the upper half's best goes through LDS (xs is free) and
             * is merged in row-tile order, which keeps the first maximum */
            float* const r_pv = reinterpret_cast<float*>(xs);
            int* const r_pe = reinterpret_cast<int*>(xs) + 64;
            const int sl = 16 * (wave & 3) + l16;
            float bv = 0.f;
            int be = 0;
            if (routes) {
                h8 cur[KS];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    cur[ks] = *reinterpret_cast<const h8*>(os + sl * LDS + 32 * ks + 8 * g);
                route_partial<DIM, S::RPT>(cur, s_br, g, wave >= 4 ? S::RPT : 0, rfrag, bv, be);
                if (wave >= 4 && g == 0) {
                    r_pv[sl] = bv;
                    r_pe[sl] = be;
                }
            }
            __syncthreads();
            if (wave < 4 && routes) {
                float v;
                int e;
                route_pick(bv, be, r_pv[sl], r_pe[sl], v, e);
                if (e >= a.n_experts || e < 0) e = 0; /* non-finite logits */
                const int sy = wy * 8 + (sl >> 3), sx = wxx * 8 + (sl & 7);
                if (g == 0) {
                    r_e[sl] = e;
                    r_rank[sl] = (sy < a.H && sx < a.W) ? atomicAdd(&r_hist[e], 1) : 0;
                }
            }
        } else if (routes) { /* wave w: tokens 16w..16w+15, all experts */
            const int sl = 16 * wave + l16;
            const int sy = wy * 8 + (sl >> 3), sx = wxx * 8 + (sl & 7);
            h8 cur[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) cur[ks] = *reinterpret_cast<const h8*>(os + sl * LDS + 32 * ks + 8 * g);
            const int e = route_token<DIM, NPT>(cur, s_br, g, a.n_experts, rfrag);
            if (g == 0) {
                r_e[sl] = e;
                r_rank[sl] = (sy < a.H && sx < a.W) ? atomicAdd(&r_hist[e], 1) : 0;
            }
        }
        if constexpr (NW == 4) store_rows();
        __syncthreads();
        if (threadIdx.x < a.n_experts) {
            const int c = r_hist[threadIdx.x];
            r_base[threadIdx.x] = c ? atomicAdd(&a.counts[threadIdx.x * a.count_stride], c) : 0;
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            const int ty = wy * 8 + (threadIdx.x >> 3), tx = wxx * 8 + (threadIdx.x & 7);
            if (ty < a.H && tx < a.W) {
                const int token = frame * (a.H * a.W) + ty * a.W + tx;
                const int e = r_e[threadIdx.x];
                a.assign[token] = e;
                const int slot = r_base[e] + r_rank[threadIdx.x];
                if (slot < a.cap) a.perm[(int64_t)e * a.cap + slot] = token;
            }
        }
    }

    /* ---- 7. fused dense FFN (dense blocks of the d128 chain): the window's
     * y rows are the FFN block's input h, already in os. The same
     * arithmetic in the same order as the expert kernel's dense path
     * (moe_expert_skip.comp.glsl:25-54 for expert 0): hn = r16(LN2(h)) (the
     * affine folded into W1/b1), u = r16(W1 hn + b1), g = r16(GELU(u)),
     * y2 = r16(W2 g + b2), out = y2 + h in fp16, so the output equals the
     * attention launch followed by the expert launch bit for bit. */
    if constexpr (FFN) {
        static_assert(NPT == 0, "dense blocks only");
        constexpr int RT = DIM / 16 / NW; /* hidden / output row tiles per wave */
        static_assert(RT >= 1, "FFN shape");
        const FragSrc w1(a.ffn_w1, DIM * DIM * 2u), w2(a.ffn_w2, DIM * DIM * 2u);
        /* the wave's weight stream: W1 then W2, k-step-major over its RT row
         * tiles, through a ring of FR fragments (all of W1 when that is at
         * most 16 fragments, W2 then refilling the slots GEMM1 frees; else
         * 3 k-steps ahead) */
        constexpr int NFF = 2 * RT * KS;
        constexpr int FR = RT * KS <= 16 ? RT * KS : 3 * RT;
        auto ffrag = [&](int p) -> h8 {
            const int q = p % (RT * KS), ks = q / RT, r = q % RT;
            return (p < RT * KS ? w1 : w2).load((wave * RT + r) * KS + ks, loff);
        };
        h8 wf[FR];
#pragma unroll
        for (int p = 0; p < FR; ++p) wf[p] = ffrag(p);
        /* LN2 of the window's slots into xs (dead since the out-projection),
         * the rows each wave normalised in LN1 */
        if (lnw) {
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const int row = (wave * SPW + it * SPI + lane / LPS) * LDS;
                const int ca = (lane % LPS) * 8;
                const RowChunk hr{*reinterpret_cast<const h8*>(os + row + ca),
                                  *reinterpret_cast<const h8*>(os + row + ca + DIM / 2)};
                ln_store<DIM>(hr, valid[it], xs + row, nullptr);
            }
        }
        __syncthreads();
        f4 facc[RT][4]; /* starts at b1 */
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const int ch = (wave * RT + r) * 16 + 4 * g;
            const f4 bb = {a.ffn_b1[ch], a.ffn_b1[ch + 1], a.ffn_b1[ch + 2], a.ffn_b1[ch + 3]};
#pragma unroll
            for (int t = 0; t < 4; ++t) facc[r][t] = bb;
        }
        h8 ff[4], fn[4];
#pragma unroll
        for (int t = 0; t < TQ; ++t) ff[t] = *reinterpret_cast<const h8*>(xs + (16 * t + l16) * LDS + 8 * g);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if (ks + 1 < KS) {
#pragma unroll
                for (int t = 0; t < TQ; ++t)
                    fn[t] = *reinterpret_cast<const h8*>(xs + (16 * t + l16) * LDS + 32 * (ks + 1) + 8 * g);
            }
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const int p = ks * RT + r;
#pragma unroll
                for (int t = 0; t < TQ; ++t) facc[r][t] = mfma_16x16x32(wf[p % FR], ff[t], facc[r][t]);
                if (p + FR < NFF) wf[p % FR] = ffrag(p + FR);
            }
            if (ks + 1 < KS) {
#pragma unroll
                for (int t = 0; t < TQ; ++t) ff[t] = fn[t];
            }
            sched_fence();
        }
        __syncthreads(); /* every wave is done reading the LN2 tile */
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const int ch = (wave * RT + r) * 16 + 4 * g;
            const f4 bb = {a.ffn_b2[ch], a.ffn_b2[ch + 1], a.ffn_b2[ch + 2], a.ffn_b2[ch + 3]};
#pragma unroll
            for (int t = 0; t < TQ; ++t) {
                const h4 u = cvt_h4(facc[r][t]); /* r16(W1 hn + b1) */
                f4 gl;
#pragma unroll
                for (int i = 0; i < 4; ++i) gl[i] = gelu_tanh_h(u[i]);
                *reinterpret_cast<h4*>(xs + (16 * t + l16) * LDS + ch) = cvt_h4(gl);
                facc[r][t] = bb; /* GEMM2 starts at b2 */
            }
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < TQ; ++t) ff[t] = *reinterpret_cast<const h8*>(xs + (16 * t + l16) * LDS + 8 * g);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if (ks + 1 < KS) {
#pragma unroll
                for (int t = 0; t < TQ; ++t)
                    fn[t] = *reinterpret_cast<const h8*>(xs + (16 * t + l16) * LDS + 32 * (ks + 1) + 8 * g);
            }
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const int p = RT * KS + ks * RT + r;
#pragma unroll
                for (int t = 0; t < TQ; ++t) facc[r][t] = mfma_16x16x32(wf[p % FR], ff[t], facc[r][t]);
                if (p + FR < NFF) wf[p % FR] = ffrag(p + FR);
            }
            if (ks + 1 < KS) {
#pragma unroll
                for (int t = 0; t < TQ; ++t) ff[t] = fn[t];
            }
            sched_fence();
        }
        /* out = r16(W2 g + b2) + h in fp16, over h in os (every residual read
           before the first add) */
        h4 hres[4][RT];
#pragma unroll
        for (int t = 0; t < TQ; ++t)
#pragma unroll
            for (int r = 0; r < RT; ++r)
                hres[t][r] = *reinterpret_cast<const h4*>(os + (16 * t + l16) * LDS + (wave * RT + r) * 16 + 4 * g);
#pragma unroll
        for (int t = 0; t < TQ; ++t)
#pragma unroll
            for (int r = 0; r < RT; ++r)
                *reinterpret_cast<h4*>(os + (16 * t + l16) * LDS + (wave * RT + r) * 16 + 4 * g) =
                    add_f16x4(cvt_h4(facc[r][t]), hres[t][r]);
        __syncthreads(); /* the block's output tile complete in os */
    }

    if constexpr (NPT == 0 || NW == 8) store_rows();
}

template <int DIM, int HD, int NW, int NPT, bool FFN = false>
__device__ __forceinline__ void attn_window(const AttnArgs& a, AttnLds<DIM, NPT>& L) {
    const int wi = blockIdx.x % a.windows_per_frame;
    const int wy = wi / a.wx, wxx = wi - (wi / a.wx) * a.wx;
    const int lane = lane_id();
    const unsigned long long vmask = __ballot(wy * 8 + (lane >> 3) < a.H && wxx * 8 + (lane & 7) < a.W);
    const bool half = (vmask >> 32) == 0ull; /* uniform */
    if (a.bqkv_pad != nullptr && vmask != ~0ull) {
        if (half)
            attn_window_body<DIM, HD, NW, NPT, true, true, FFN>(a, L, vmask);
        else
            attn_window_body<DIM, HD, NW, NPT, true, false, FFN>(a, L, vmask);
    } else if (half) {
        attn_window_body<DIM, HD, NW, NPT, false, true, FFN>(a, L, vmask);
    } else {
        attn_window_body<DIM, HD, NW, NPT, false, false, FFN>(a, L, vmask);
    }
}

/* 4 waves (2 heads each, 2 workgroups per CU) for large grids; 8 waves (one
 * head each, one workgroup per CU) when windows are scarcer than CUs. The
 * _r<NPT> kernels also route the window's tokens (16*NPT padded experts). */
#define PRISM_ATTN_KERNELS(D, HD, NPT, SUF)                                                          \
    extern "C" __global__ void __launch_bounds__(256, 2) prism_attn_d##D##SUF(AttnArgs a) {          \
        __shared__ AttnLds<D, NPT> lds;                                                              \
        attn_window<D, HD, 4, NPT>(a, lds);                                                          \
    }                                                                                                \
    extern "C" __global__ void __launch_bounds__(512, 1) prism_attn_d##D##_w8##SUF(AttnArgs a) {     \
        __shared__ AttnLds<D, NPT> lds;                                                              \
        attn_window<D, HD, 8, NPT>(a, lds);                                                          \
    }
PRISM_ATTN_KERNELS(256, 32, 0, )
PRISM_ATTN_KERNELS(256, 32, 1, _r1)
PRISM_ATTN_KERNELS(256, 32, 2, _r2)
PRISM_ATTN_KERNELS(256, 32, 3, _r3)
PRISM_ATTN_KERNELS(256, 32, 4, _r4)
PRISM_ATTN_KERNELS(128, 16, 0, )
PRISM_ATTN_KERNELS(128, 16, 1, _r1)
PRISM_ATTN_KERNELS(128, 16, 2, _r2)
PRISM_ATTN_KERNELS(128, 16, 3, _r3)
PRISM_ATTN_KERNELS(128, 16, 4, _r4)

/* dense blocks in the chain: attention with the block's FFN fused (the
 * chain's one launch per dense block) */
extern "C" __global__ void __launch_bounds__(256, 2) prism_attn_d128_ffn(AttnArgs a) {
    __shared__ AttnLds<128, 0> lds;
    attn_window<128, 16, 4, 0, true>(a, lds);
}
extern "C" __global__ void __launch_bounds__(512, 1) prism_attn_d128_w8_ffn(AttnArgs a) {
    __shared__ AttnLds<128, 0> lds;
    attn_window<128, 16, 8, 0, true>(a, lds);
}
extern "C" __global__ void __launch_bounds__(256, 2) prism_attn_d256_ffn(AttnArgs a) {
    __shared__ AttnLds<256, 0> lds;
    attn_window<256, 32, 4, 0, true>(a, lds);
}
extern "C" __global__ void __launch_bounds__(512, 1) prism_attn_d256_w8_ffn(AttnArgs a) {
    __shared__ AttnLds<256, 0> lds;
    attn_window<256, 32, 8, 0, true>(a, lds);
}
#undef PRISM_ATTN_KERNELS
