/*
 * codec.hpp - the conv encoder and fused decoder around the transformer
 * (the end-to-end frame of vulkan_engine/prism_moe_bench.cpp:387-471).
 *
 * Every stage is one implicit GEMM on fp16 MFMA, C^T = W * P^T: the packed
 * weights are the A operand (16 output channels x 32 k per fragment) and the
 * B operand is gathered per lane straight from the input maps, 16 output
 * pixels per token tile. Accumulators start at the bias; the result is
 * rounded to fp16 once (the reference rounds each 288-wide split partial
 * sum, strided_conv_split_*ch.comp.glsl:84-93, which its comments call the
 * same output), then ReLU. Maps between stages are NHWC fp16 (a pixel's
 * channels contiguous, so a lane's 8 channels are one 16-byte load); the
 * frame coming in and the display image going out are CHW, as in the
 * reference.
 *
 *   enc0  conv3x3 s1  9 -> 32  + ReLU  conv3x3_coopvec_9ch.comp.glsl:27-72
 *         (reads the CHW frame through an LDS window per 4 x 64 pixel block;
 *         k = ic*9 + tap as the reference, 81 -> 96)
 *   enc1  conv3x3 s2 32 -> 64  + ReLU  strided_conv_coopvec_32ch.comp.glsl:30-77
 *   enc2  conv3x3 s2 64 -> 128 + ReLU  strided_conv_split_64ch.comp.glsl:30-93
 *   enc3  conv3x3 s2 128-> 128 + ReLU  strided_conv_split_128ch.comp.glsl:32-94
 *         (NHWC taps: k = tap*Cin + ic; the host permutes the weight columns)
 *   dec3  NN-up(128) ++ skip e2(128) -> PW 256 -> 128 + ReLU   dec3_fused.comp.glsl:27-63
 *   dec2  NN-up(128) ++ skip e1(64)  -> PW 192 -> 64  + ReLU   dec2_fused.comp.glsl:27-55
 *   dec1  NN-up(64)  ++ skip e0(32)  -> PW 96  -> 32  + ReLU   dec1_fused.comp.glsl:27-55
 *         then PW 32 -> 12 (pw_conv_coopvec_32to12.comp.glsl:28-55) and
 *         PixelShuffle(2) + sigmoid (pixelshuffle_sigmoid.comp.glsl:28-56)
 *         in the same kernel: dec1's accumulator lanes hold channels
 *         4g..4g+3 and 16+4g..16+4g+3 of their pixel, which is a B fragment
 *         of the 32 -> 12 GEMM under the permuted k numbering
 *         k(g, j) = 16*(j/4) + 4g + j%4 (the host packs that weight with its
 *         columns permuted to match). The 12 channels round to fp16 (the
 *         reference's out12 map), then sigmoid in fp32, fp16 again, written
 *         as 2x2 display pixels of the lane's RGB plane.
 *
 * Workgroup = 4 waves; a wave takes TT consecutive 16-pixel tiles (pixels in
 * row-major order of the output map, blockIdx.y = frame) and all COUT output
 * channels, or 1/RS of them (channel split), or all of them over 1/KSP of
 * the reduction (K-split, enc3). Each k-step's weight fragments and B
 * fragments are loaded one
 * k-step ahead of its MFMAs. Loads at padded or out-of-map positions return
 * zeros through the input buffer's range check (MapSrc).
 */
#pragma once
#include "common.hpp"

/* Output pixel of one lane in one token tile. */
struct CodecPix {
    int y, x;
    bool valid;
};

/* The B gathers read a frame's map through a buffer resource whose range is
 * the map: a lane whose operand is zero (a tap in the conv padding) or
 * unused (a pixel past the map's end, whose output column is never stored)
 * gets the offset CODEC_OOB, and the range check returns zeros for it. Each
 * lane's byte offsets are 32-bit (the host keeps a frame's largest map under
 * 2 GiB) and computed once per token tile, so a load is one instruction with
 * its k-step's channel offset in the immediate field. */
static constexpr uint32_t CODEC_OOB = 0x80000000u;
struct MapSrc {
    __amdgpu_buffer_rsrc_t r;
    __device__ __forceinline__ MapSrc(const uint16_t* base, uint32_t bytes)
        : r(__builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000)) {}
    __device__ __forceinline__ h8 load(uint32_t off) const {
        return __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    }
};

/* conv3x3 (pad 1) over an NHWC map with CIN channels; k = tap*CIN + ic. A
 * tile's per-lane state: the byte offset of each of the 9 taps' input pixel
 * (channel 8g), CODEC_OOB where the tap falls in the padding. */
template <int CIN, int STRIDE>
struct SrcConvNHWC {
    static constexpr int KS = 9 * CIN / 32;
    MapSrc m;
    int iw, ih;
    struct Pix {
        uint32_t off[9];
    };
    __device__ __forceinline__ Pix prep(const CodecPix& p, int g) const {
        Pix q;
        const int iy0 = p.y * STRIDE - 1, ix0 = p.x * STRIDE - 1;
        const int base = ((iy0 * iw + ix0) * CIN + 8 * g) * 2; /* may be negative: only in-map taps use it */
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            const int iy = iy0 + tap / 3, ix = ix0 + tap % 3;
            const bool ok = p.valid && iy >= 0 && iy < ih && ix >= 0 && ix < iw;
            q.off[tap] = ok ? (uint32_t)(base + ((tap / 3) * iw + tap % 3) * CIN * 2) : CODEC_OOB;
        }
        return q;
    }
    /* k-step i KSP + j (i compile-time, j < KSP wave-uniform) */
    template <int KSP>
    __device__ __forceinline__ h8 load(int i, int j, const Pix& q) const {
        constexpr int CPT = CIN / 32; /* k-steps per tap */
        static_assert(CPT % KSP == 0, "a split's k-steps stay within one tap");
        return m.load(q.off[i * KSP / CPT] + (uint32_t)(((i * KSP) % CPT + j) * 64));
    }
};

/* Decoder input: channels [0, CUP) from the NN-upsampled coarse map (pixel
 * (min(y/2, uh-1), min(x/2, uw-1))), then [CUP, CUP+CSKIP) from the skip map
 * at the same pixel. */
template <int CUP, int CSKIP>
struct SrcDec {
    static constexpr int KS = (CUP + CSKIP) / 32;
    MapSrc mu, ms;
    int uw, uh, ow;
    struct Pix {
        uint32_t up, skip;
    };
    __device__ __forceinline__ Pix prep(const CodecPix& p, int g) const {
        const int uy = min(p.y >> 1, uh - 1), ux = min(p.x >> 1, uw - 1);
        return Pix{p.valid ? (uint32_t)(((uy * uw + ux) * CUP + 8 * g) * 2) : CODEC_OOB,
                   p.valid ? (uint32_t)(((p.y * ow + p.x) * CSKIP + 8 * g) * 2) : CODEC_OOB};
    }
    /* k-step i KSP + j (i compile-time, j < KSP wave-uniform) */
    template <int KSP>
    __device__ __forceinline__ h8 load(int i, int j, const Pix& q) const {
        static_assert((CUP / 32) % KSP == 0, "a split's k-steps stay within one map");
        if (32 * i * KSP < CUP) return mu.load(q.up + (uint32_t)(64 * (i * KSP + j)));
        return ms.load(q.skip + (uint32_t)(64 * (i * KSP + j) - 2 * CUP));
    }
};

/* The GEMM: acc[r][t] = bias + W[16(rt0 + r).., :] * P[:, tile t] for RT row
 * tiles from rt0 (of the matrix's RTALL), over the k-steps i KSP + kj
 * (all of them for KSP = 1; a K-split stage's wave kj takes every KSP-th,
 * and only kj = 0 starts at the bias). */
template <class Src, int RTALL, int RT, int TT, int KSP = 1>
__device__ __forceinline__ void codec_gemm(const Src& src, const uint16_t* w, const float* bias, const CodecPix (&px)[TT],
                                           int g, int lane, int rt0, f4 (&acc)[RT][TT], int kj = 0) {
    constexpr int KS = Src::KS, KN = KS / KSP;
    static_assert(KS % KSP == 0, "whole k-steps per wave");
    const FragSrc wsrc(w, (unsigned)(RTALL * KS * 1024));
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int ch = 16 * (rt0 + r) + 4 * g;
        const f4 bb = kj == 0 ? f4{bias[ch], bias[ch + 1], bias[ch + 2], bias[ch + 3]} : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = bb;
    }
    typename Src::Pix q[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) q[t] = src.prep(px[t], g);
    h8 bc[TT], bn[TT], wc[RT], wn[RT];
#pragma unroll
    for (int t = 0; t < TT; ++t) bc[t] = src.template load<KSP>(0, kj, q[t]);
#pragma unroll
    for (int r = 0; r < RT; ++r) wc[r] = wsrc.load((rt0 + r) * KS + kj, lane * 16);
#pragma unroll
    for (int ks = 0; ks < KN; ++ks) {
        if (ks + 1 < KN) {
#pragma unroll
            for (int t = 0; t < TT; ++t) bn[t] = src.template load<KSP>(ks + 1, kj, q[t]);
#pragma unroll
            for (int r = 0; r < RT; ++r) wn[r] = wsrc.load((rt0 + r) * KS + (ks + 1) * KSP + kj, lane * 16);
        }
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int t = 0; t < TT; ++t) acc[r][t] = mfma_16x16x32(wc[r], bc[t], acc[r][t]);
        if (ks + 1 < KN) {
#pragma unroll
            for (int t = 0; t < TT; ++t) bc[t] = bn[t];
#pragma unroll
            for (int r = 0; r < RT; ++r) wc[r] = wn[r];
        }
        sched_fence();
    }
}

/* The pixel block a workgroup takes: workgroups are dealt to the 8 XCDs in
 * turn (workgroup b to XCD b % 8), each with its own L2, so consecutive
 * blocks (which share input rows: the conv taps' halo, the stride-2 rows
 * between two output rows, the decoder's upsampled rows) go to the same XCD
 * in a contiguous band of about 1/8 of the map: the first n % 8 XCDs take
 * n/8 + 1 blocks, the others n/8 (a permutation of [0, n), whatever the
 * hardware's actual placement). BAND = false keeps the launch order: the
 * decoder's dec3 and dec1 and the small enc3 run faster with every XCD
 * sweeping the map top to bottom together (enc0, enc1, enc2, dec2 faster
 * banded: 1.7, 1.6, 0.5, 0.2 us at 960x540; dec1, dec3, enc3 0.4, 0.2,
 * 0.1 us slower). */
template <bool BAND>
__device__ __forceinline__ int codec_block() {
    if constexpr (!BAND) return (int)blockIdx.x;
    const int n = (int)gridDim.x, b = (int)blockIdx.x;
    const int q = n >> 3, r = n & 7, x = b & 7, j = b >> 3;
    return x < r ? x * (q + 1) + j : r * (q + 1) + (x - r) * q + j;
}

/* A workgroup's output block from LDS to memory in 16-byte chunks (NPX
 * pixels of CPP chunks, NT threads). Every LDS read is issued before the
 * first store: a read under a store's condition costs one LDS round trip per
 * pass. src(pl): the LDS address of block pixel pl's first channel; dst(pl):
 * the memory address of its first channel, or nullptr past the map. */
template <int NPX, int CPP, int NT, class Src, class Dst>
__device__ __forceinline__ void codec_store_block(Src&& src, Dst&& dst) {
    constexpr int N = NPX * CPP, IT = (N + NT - 1) / NT;
    h8 v[IT];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int q = min((int)threadIdx.x + NT * it, N - 1);
        v[it] = *reinterpret_cast<const h8*>(src(q / CPP) + (q % CPP) * 8);
    }
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int q = (int)threadIdx.x + NT * it;
        if (q < N) {
            uint16_t* d = dst(q / CPP);
            if (d) *reinterpret_cast<h8*>(d + (q % CPP) * 8) = v[it];
        }
    }
}

/* A workgroup's 4 waves form 4/RS pixel groups of TT tiles each; the RS waves
 * of a group split the output channels. */
template <int TT, int RS, bool BAND>
__device__ __forceinline__ void codec_pixels(const CodecArgs& a, int wave, int l16, CodecPix (&px)[TT]) {
    const int npix = a.out_w * a.out_h;
    const int p0 = (codec_block<BAND>() * (4 / RS) + wave / RS) * TT * 16;
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const int p = p0 + 16 * t + l16;
        px[t].valid = p < npix;
        const int q = px[t].valid ? p : 0;
        px[t].y = q / a.out_w;
        px[t].x = q - px[t].y * a.out_w;
    }
}

/* One stage: GEMM, ReLU, fp16, NHWC store. The workgroup's pixels are
 * consecutive, so its output is one contiguous block: the tile is assembled
 * in LDS and leaves as whole pixel rows, 16 bytes per lane (a store straight
 * from the accumulators writes 16 pixels x 32 bytes per instruction). */
template <class Src, int COUT, int TT, int RS, bool BAND>
__device__ __forceinline__ void codec_stage(const CodecArgs& a, const Src& src) {
    constexpr int RTALL = COUT / 16, RT = RTALL / RS;
    static_assert(COUT % 16 == 0 && RTALL % RS == 0 && 4 % RS == 0, "whole row tiles");
    constexpr int NPX = (4 / RS) * TT * 16, LDO = COUT + 8; /* pixels per workgroup, padded LDS row */
    __shared__ __attribute__((aligned(16))) f16 otile[NPX * LDO];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    CodecPix px[TT];
    codec_pixels<TT, RS, BAND>(a, wave, l16, px);
    const int rt0 = (wave % RS) * RT;
    f4 acc[RT][TT];
    codec_gemm<Src, RTALL, RT, TT>(src, a.w, a.b, px, g, lane, rt0, acc);
    const int pl0 = (wave / RS) * TT * 16; /* this wave's first pixel in the workgroup's block */
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            f4 v = acc[r][t];
            /* max(r16(v), 0) == r16(max(v, 0)): fp16 rounding is monotonic */
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = fmaxf(v[i], 0.f);
            *reinterpret_cast<h4*>(otile + (pl0 + 16 * t + l16) * LDO + 16 * (rt0 + r) + 4 * g) = cvt_h4(v);
        }
    __syncthreads();
    const int64_t p0 = (int64_t)codec_block<BAND>() * NPX, npix = (int64_t)a.out_w * a.out_h;
    uint16_t* out = a.out + (int64_t)blockIdx.y * a.out_frame;
    codec_store_block<NPX, COUT / 8, 256>([&](int pl) { return otile + pl * LDO; },
                                          [&](int pl) { return p0 + pl < npix ? out + (p0 + pl) * COUT : nullptr; });
}

/* One stage with its reduction split over KSP waves (K-split): the
 * workgroup's 4 waves form 4/KSP pixel groups of TT tiles; wave j of a group
 * takes every KSP-th k-step from j for every output channel, so each wave's
 * chain of dependent weight and operand round trips is KSP times shorter
 * than the whole reduction (the deep stages' reductions are latency chains
 * otherwise: few MFMAs per k-step, one round trip each). Wave j then owns
 * row tiles [j RQ, (j+1) RQ) (RQ = RTALL/KSP): it publishes its partial
 * tiles of the other rows in LDS, sums the group's KSP partials of its own
 * rows in wave order (the first carries the bias), ReLU, fp16, into the
 * output tile. */
/* The K-split reduction: wave `wave`, position kq = wave % KSP of pixel
 * group wave / KSP, holds partial sums of all RTALL row tiles over its
 * k-steps (acc); it publishes those of the rows it does not own in `part`
 * ([wave][row tile not owned][t][lane]), then sums the group's KSP partials
 * of its own RQ = RTALL / KSP rows from kq RQ in wave order (the first
 * carries the bias): ReLU, fp16, into the output tile (pixel row
 * pg TT 16 + 16 t + l16, LDO halfs a row). One workgroup barrier, between
 * publishing and summing. */
template <int RTALL, int TT, int KSP, int LDO>
__device__ __forceinline__ void codec_ksplit_reduce(const f4 (&accin)[RTALL][TT], f4* part, f16* otile, int wave,
                                                    int lane, int l16, int g) {
    constexpr int RQ = RTALL / KSP, NO = RTALL - RQ;
    f4 acc[RTALL][TT]; /* a local copy: selected from below without indexing registers */
#pragma unroll
    for (int r = 0; r < RTALL; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = accin[r][t];
    const int pg = wave / KSP, kq = wave % KSP;
    /* the slot of row tile r (not owned by position j) of wave w; for an owned
     * r (a value the reduction computes and does not use) a slot in range */
    auto slot = [&](int w, int j, int r, int t) {
        return ((w * NO + (r < j * RQ ? r : max(r - RQ, 0))) * TT + t) * 64 + lane;
    };
#pragma unroll
    for (int r = 0; r < RTALL; ++r)
        if (r / RQ != kq) /* uniform */
#pragma unroll
            for (int t = 0; t < TT; ++t) part[slot(wave, kq, r, t)] = acc[r][t];
    __syncthreads();
    const int pl0 = pg * TT * 16;
    /* kq with its range hidden: knowing kq < KSP, the compiler turns the
     * select chain below into a register index (private memory) */
    int ksel = kq;
    asm("" : "+s"(ksel));
#pragma unroll
    for (int rr = 0; rr < RQ; ++rr) {
        const int r = kq * RQ + rr;
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            f4 own = acc[rr][t]; /* acc[r][t], selected without indexing registers */
#pragma unroll
            for (int c = 1; c < KSP; ++c)
                if (ksel == c) own = acc[c * RQ + rr][t];
            f4 v = kq == 0 ? own : part[slot(pg * KSP, 0, r, t)];
#pragma unroll
            for (int j = 1; j < KSP; ++j) {
                const f4 u = kq == j ? own : part[slot(pg * KSP + j, j, r, t)];
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] += u[i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = fmaxf(v[i], 0.f);
            *reinterpret_cast<h4*>(otile + (pl0 + 16 * t + l16) * LDO + 16 * r + 4 * g) = cvt_h4(v);
        }
    }
}

template <class Src, int COUT, int TT, int KSP, bool BAND>
__device__ __forceinline__ void codec_stage_ksplit(const CodecArgs& a, const Src& src) {
    constexpr int RTALL = COUT / 16, RQ = RTALL / KSP, NO = RTALL - RQ;
    static_assert(COUT % 16 == 0 && 4 % KSP == 0 && RTALL % KSP == 0, "K-split shape");
    constexpr int NPX = (4 / KSP) * TT * 16, LDO = COUT + 8;
    __shared__ __attribute__((aligned(16))) f4 part[4 * NO * TT * 64]; /* [wave][row tile not owned][t][lane] */
    __shared__ __attribute__((aligned(16))) f16 otile[NPX * LDO];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    CodecPix px[TT];
    codec_pixels<TT, KSP, BAND>(a, wave, l16, px);
    f4 acc[RTALL][TT];
    codec_gemm<Src, RTALL, RTALL, TT, KSP>(src, a.w, a.b, px, g, lane, 0, acc, wave % KSP);
    codec_ksplit_reduce<RTALL, TT, KSP, LDO>(acc, part, otile, wave, lane, l16, g);
    __syncthreads();
    const int64_t p0 = (int64_t)codec_block<BAND>() * NPX, npix = (int64_t)a.out_w * a.out_h;
    uint16_t* out = a.out + (int64_t)blockIdx.y * a.out_frame;
    codec_store_block<NPX, COUT / 8, 256>([&](int pl) { return otile + pl * LDO; },
                                          [&](int pl) { return p0 + pl < npix ? out + (p0 + pl) * COUT : nullptr; });
}

/* A stage's kernel body: K-split when KSP > 1, else channels split over RS
 * waves. */
template <class Src, int COUT, int TT, int RS, int KSP, bool BAND>
__device__ __forceinline__ void codec_stage_any(const CodecArgs& a, const Src& src) {
    static_assert(RS == 1 || KSP == 1, "a stage splits its channels or its reduction, not both");
    if constexpr (KSP > 1) codec_stage_ksplit<Src, COUT, TT, KSP, BAND>(a, src);
    else codec_stage<Src, COUT, TT, RS, BAND>(a, src);
}

/* dec1's output tiles (acc: its 32 channels, bias in) -> ReLU, fp16, the
 * 32 -> 12 conv, fp16, sigmoid, fp16, PixelShuffle(2) into the CHW display. */
template <int TT>
__device__ __forceinline__ void codec_out_shuffle(const CodecArgs& a, const CodecPix (&px)[TT], const f4 (&acc)[2][TT],
                                                  int g, int lane) {
    const int f = blockIdx.y;
    /* the 32 -> 12 weights: one fragment (rows 12..15 zero), columns permuted */
    const h8 wo = FragSrc(a.w2, 1024u).load(0, lane * 16);
    const f4 bo = {a.b2[4 * g], a.b2[4 * g + 1], a.b2[4 * g + 2], a.b2[4 * g + 3]};
    constexpr float LOG2E = 1.4426950408889634f;
    const int dw = 2 * a.out_w, dh = 2 * a.out_h;
    uint16_t* disp = a.out + (int64_t)f * a.out_frame;
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        h4 y[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            f4 v = acc[r][t];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = fmaxf(v[i], 0.f);
            y[r] = cvt_h4(v); /* dec1 output, r16 + ReLU */
        }
        const h8 yb = {y[0][0], y[0][1], y[0][2], y[0][3], y[1][0], y[1][1], y[1][2], y[1][3]};
        const h4 o12 = cvt_h4(mfma_16x16x32(wo, yb, bo)); /* out12 channels 4g..4g+3 */
        if (!px[t].valid || g == 3) continue;             /* rows 12..15 are padding */
        h4 s;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = (float)o12[i];
            s[i] = (_Float16)fast_rcp(1.0f + fast_exp2(-v * LOG2E));
        }
        /* channel 4g + 2sy + sx -> RGB plane g, display pixel (2y + sy, 2x + sx) */
        uint16_t* base = disp + ((int64_t)g * dh + 2 * px[t].y) * dw + 2 * px[t].x;
        const uint32_t top = __builtin_bit_cast(uint32_t, __builtin_shufflevector(s, s, 0, 1));
        const uint32_t bot = __builtin_bit_cast(uint32_t, __builtin_shufflevector(s, s, 2, 3));
        *reinterpret_cast<uint32_t*>(base) = top;
        *reinterpret_cast<uint32_t*>(base + dw) = bot;
    }
}

/* dec1 + output conv + PixelShuffle(2) + sigmoid. */
template <int TT>
__device__ __forceinline__ void codec_dec_out(const CodecArgs& a) {
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    CodecPix px[TT];
    codec_pixels<TT, 1, false>(a, wave, l16, px);
    const int f = blockIdx.y;
    const SrcDec<64, 32> src{MapSrc(a.in + (int64_t)f * a.in_frame, (uint32_t)(a.in_frame * 2)),
                             MapSrc(a.skip + (int64_t)f * a.skip_frame, (uint32_t)(a.skip_frame * 2)), a.in_w, a.in_h,
                             a.out_w};
    f4 acc[2][TT];
    codec_gemm<SrcDec<64, 32>, 2, 2, TT>(src, a.w, a.b, px, g, lane, 0, acc);
    codec_out_shuffle<TT>(a, px, acc, g, lane);
}

/* Decoder input read by the fused dec2 + dec1 kernel: channels [0, 64) from
 * the workgroup's LDS block of the dec2 output (the NN-upsampled coarse map:
 * r1 pixel (y/2, x/2), relative to the block's origin (y1, x1); LDS rows of
 * LD halfs), [64, 96) from the e0 skip map at the same pixel. */
struct SrcDecLds {
    static constexpr int KS = 3, CUP = 64, CSKIP = 32, LD = 64 + 8, C1 = 32;
    const f16* lds;
    MapSrc ms;
    int ow, y1, x1;
    struct Pix {
        uint32_t up, skip;
    };
    __device__ __forceinline__ Pix prep(const CodecPix& p, int g) const {
        /* an invalid pixel reads the block's first row: in LDS, never used */
        const int loc = p.valid ? ((p.y >> 1) - y1) * C1 + ((p.x >> 1) - x1) : 0;
        return Pix{(uint32_t)((loc * LD + 8 * g) * 2),
                   p.valid ? (uint32_t)(((p.y * ow + p.x) * CSKIP + 8 * g) * 2) : CODEC_OOB};
    }
    template <int KSP>
    __device__ __forceinline__ h8 load(int i, int j, const Pix& q) const {
        static_assert(KSP == 1, "no K-split");
        if (32 * i < CUP)
            return *reinterpret_cast<const h8*>(reinterpret_cast<const unsigned char*>(lds) + q.up + 64 * i);
        return ms.load(q.skip + (uint32_t)(64 * i - 2 * CUP));
    }
};

/* dec2 + dec1 + output conv + PixelShuffle(2) + sigmoid in one launch. Both
 * decoder stages are pointwise after a nearest-neighbour upsample, so an
 * r0 block of 4 x 64 pixels needs exactly the r1 block of 2 x 32 pixels
 * under it: the workgroup computes that dec2 block (wave w: r1 row w/2,
 * columns 16(w%2)..+15, all 64 channels; the same fragments, k order,
 * rounding and ReLU as prism_codec_dec2) into LDS, then dec1 and the output
 * for its r0 block (wave w: r0 row w, 4 tiles of 16 columns) with the
 * upsampled channels read from LDS. The dec2 map never reaches memory; the
 * output equals the two separate launches bit for bit. Grid: x =
 * ceil(w1/32) * ceil(h1/2) blocks, y = frames. a2: dec2's arguments (in =
 * the dec3 map, skip = e1, out unused); a1: dec1's (in unused, skip = e0,
 * out = the display). */
__device__ __forceinline__ void codec_dec21_out(const CodecArgs& a2, const CodecArgs& a1) {
    constexpr int C1 = SrcDecLds::C1, LD = SrcDecLds::LD;
    __shared__ __attribute__((aligned(16))) f16 d2s[2 * C1 * LD];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int f = blockIdx.y;
    const int w1 = a2.out_w, h1 = a2.out_h, bxn = (w1 + C1 - 1) / C1;
    const int y1 = (blockIdx.x / bxn) * 2, x1 = (blockIdx.x % bxn) * C1;
    /* ---- dec2 for the r1 block, into LDS */
    {
        CodecPix px[1];
        px[0].y = y1 + (wave >> 1);
        px[0].x = x1 + 16 * (wave & 1) + l16;
        px[0].valid = px[0].y < h1 && px[0].x < w1;
        const SrcDec<128, 64> src{MapSrc(a2.in + (int64_t)f * a2.in_frame, (uint32_t)(a2.in_frame * 2)),
                                  MapSrc(a2.skip + (int64_t)f * a2.skip_frame, (uint32_t)(a2.skip_frame * 2)),
                                  a2.in_w, a2.in_h, w1};
        f4 acc[4][1];
        codec_gemm<SrcDec<128, 64>, 4, 4, 1>(src, a2.w, a2.b, px, g, lane, 0, acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            f4 v = acc[r][0];
            /* max(r16(v), 0) == r16(max(v, 0)): fp16 rounding is monotonic */
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = fmaxf(v[i], 0.f);
            *reinterpret_cast<h4*>(d2s + (16 * wave + l16) * LD + 16 * r + 4 * g) = cvt_h4(v);
        }
    }
    __syncthreads();
    /* ---- dec1 + output for the r0 block */
    constexpr int TT = 4;
    CodecPix px[TT];
    const int w0 = a1.out_w, h0 = a1.out_h;
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        px[t].y = 2 * y1 + wave;
        px[t].x = 2 * x1 + 16 * t + l16;
        px[t].valid = px[t].y < h0 && px[t].x < w0;
    }
    const SrcDecLds src{d2s, MapSrc(a1.skip + (int64_t)f * a1.skip_frame, (uint32_t)(a1.skip_frame * 2)), w0, y1, x1};
    f4 acc[2][TT];
    codec_gemm<SrcDecLds, 2, 2, TT>(src, a1.w, a1.b, px, g, lane, 0, acc);
    codec_out_shuffle<TT>(a1, px, acc, g, lane);
}

/* An NHWC map's window (WR x WC pixels of CIN channels from pixel (gy0, gx0))
 * into LDS, LDE halfs a pixel, zeros where it leaves the map, by NT threads.
 * Every load of a thread is issued before its first LDS store, so the window
 * costs one memory round trip (a loop with a guarded load and a store per
 * pass costs one per pass); loads outside the map read zero through the
 * buffer resource. */
template <int CIN, int WR, int WC, int LDE, int NT>
__device__ __forceinline__ void codec_map_window(const MapSrc& m, int W, int H, int gy0, int gx0, f16* lds) {
    constexpr int CPP = CIN / 8, N = WR * WC * CPP, IT = (N + NT - 1) / NT;
    h8 v[IT];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int q = (int)threadIdx.x + NT * it;
        const int px = q / CPP, c8 = (q - px * CPP) * 8;
        const int r = px / WC, c = px - r * WC;
        const int gy = gy0 + r, gx = gx0 + c;
        const bool ok = q < N && gy >= 0 && gy < H && gx >= 0 && gx < W;
        v[it] = m.load(ok ? (uint32_t)(((gy * W + gx) * CIN + c8) * 2) : CODEC_OOB);
    }
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int q = (int)threadIdx.x + NT * it;
        const int px = q / CPP, c8 = (q - px * CPP) * 8;
        if (q < N) *reinterpret_cast<h8*>(lds + px * LDE + c8) = v[it];
    }
}

/* The frame window under a block: FR x FC pixels of the 9-channel CHW frame
 * from pixel (gy0, gx0), into LDS as 16 halfs a pixel (channels 9-15 zero;
 * zeros where the window leaves the frame), by 256 threads. Every load of a
 * thread is issued before its first LDS store, so the window costs one memory
 * round trip; a load for a pixel outside the frame reads pixel 0, and its
 * value is replaced by zero. */
template <int FR, int FC>
__device__ __forceinline__ void codec_frame_window(const f16* frame, int W0, int H0, int gy0, int gx0, f16* s_in) {
    constexpr int NPX = FR * FC, IT = (NPX + 255) / 256, CH = 9, CP = 16;
    const int64_t plane = (int64_t)W0 * H0;
    f16 v[IT][CH];
    bool ok[IT];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int px = min((int)threadIdx.x + 256 * it, NPX - 1);
        const int r = px / FC, x = px - r * FC;
        const int gy = gy0 + r, gx = gx0 + x;
        ok[it] = gy >= 0 && gy < H0 && gx >= 0 && gx < W0;
        const f16* src = frame + (ok[it] ? (int64_t)gy * W0 + gx : 0);
#pragma unroll
        for (int c = 0; c < CH; ++c) v[it][c] = src[c * plane];
    }
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int px = threadIdx.x + 256 * it;
        if (px < NPX) {
            h8 lo, hi = {};
#pragma unroll
            for (int c = 0; c < 8; ++c) lo[c] = ok[it] ? v[it][c] : (f16)0.f;
            hi[0] = ok[it] ? v[it][8] : (f16)0.f;
            *reinterpret_cast<h8*>(s_in + px * CP) = lo;
            *reinterpret_cast<h8*>(s_in + px * CP + 8) = hi;
        }
    }
}

/* enc0: conv3x3 9 -> 32 + ReLU straight from the CHW frame. A workgroup
 * takes a block of CODEC_ENC0_ROWS x 64 output pixels (wave w: row w, 4 tiles
 * of 16 columns). The block's input window with its 1-pixel halo is first
 * copied into LDS pixel-interleaved, 16 halfs per pixel (the 9 channels, then
 * zeros), one thread per pixel; the GEMM's reduction index is then
 * k = tap * 16 + ic (9 taps x 16, padded to 160; the host packs W's stored
 * column ic * 9 + tap there), so a lane's 8 consecutive k of a k-step are
 * 8 channels of one tap: one 16-byte LDS read per B fragment. Grid: x =
 * ceil(W/CODEC_ENC0_COLS) * ceil(H/CODEC_ENC0_ROWS), y = frames. */
__device__ __forceinline__ void codec_enc0_body(const CodecArgs& a) {
    constexpr int IR = CODEC_ENC0_ROWS + 2, IC = CODEC_ENC0_COLS + 2, CH = 9, CP = 16, KS = 5,
                  TT = CODEC_ENC0_COLS / 16;
    __shared__ __attribute__((aligned(16))) f16 s_in[IR * IC * CP];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int W = a.out_w, H = a.out_h;
    const int bxn = (W + CODEC_ENC0_COLS - 1) / CODEC_ENC0_COLS;
    const int blk = codec_block<true>();
    const int by0 = (blk / bxn) * CODEC_ENC0_ROWS, bx0 = (blk % bxn) * CODEC_ENC0_COLS;
    codec_frame_window<IR, IC>(reinterpret_cast<const f16*>(a.in) + (int64_t)blockIdx.y * a.in_frame, W, H, by0 - 1,
                               bx0 - 1, s_in);
    __syncthreads();
    const FragSrc wsrc(a.w, 2u * KS * 1024u);
    f4 acc[2][TT];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int ch = 16 * r + 4 * g;
        const f4 bb = {a.b[ch], a.b[ch + 1], a.b[ch + 2], a.b[ch + 3]};
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = bb;
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const h8 w0 = wsrc.load(0 * KS + ks, lane * 16), w1 = wsrc.load(1 * KS + ks, lane * 16);
        /* k = 32 ks + 8 g + j = tap * 16 + 8 (g & 1) + j; tap 9 (the upper half
         * of the last k-step, lane groups 2 and 3) is padding: its operand is
         * zero, read from a clamped in-window address (no divergent branch
         * around the MFMAs) */
        const int tap = 2 * ks + (g >> 1), tc = tap < CH ? tap : CH - 1;
        const int ky = tc / 3, kx = tc - 3 * ky;
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            h8 b = *reinterpret_cast<const h8*>(s_in + ((wave + ky) * IC + 16 * t + l16 + kx) * CP + 8 * (g & 1));
            if (tap >= CH) b = h8{};
            acc[0][t] = mfma_16x16x32(w0, b, acc[0][t]);
            acc[1][t] = mfma_16x16x32(w1, b, acc[1][t]);
        }
    }
    const int oy = by0 + wave;
    uint16_t* out = a.out + (int64_t)blockIdx.y * a.out_frame;
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const int ox = bx0 + 16 * t + l16;
        if (oy >= H || ox >= W) continue;
        uint16_t* row = out + ((int64_t)oy * W + ox) * 32 + 4 * g;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            f4 v = acc[r][t];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = fmaxf(v[i], 0.f);
            *reinterpret_cast<h4*>(row + 16 * r) = cvt_h4(v);
        }
    }
}

/* A stride-2 conv3x3 stage over an LDS window (enc2): the workgroup takes a
 * BR x BC block of output pixels and first copies the input window under it,
 * (2 BR + 1) x (2 BC + 1) pixels of CIN channels (zeros past the map), into
 * LDS with coalesced 16-byte loads; each wave then takes a quarter of the
 * output channels over all BR x BC / 16 tiles of the block, its B fragments
 * read from the window (tap (ky, kx) of output pixel (y, x) at window pixel
 * (2 (y - oy0) + ky, 2 (x - ox0) + kx)) and its weight fragments streamed DW
 * k-steps ahead. No input tap or weight fragment is fetched by more than
 * one wave of the workgroup (the one-wave-per-pixel-group form fetches each
 * weight fragment in every wave). k order and sums as codec_stage:
 * bit-identical outputs. */
template <int CIN, int COUT, int BR, int BC, int DW, bool BAND>
__device__ __forceinline__ void codec_conv_window(const CodecArgs& a) {
    constexpr int WR = 2 * BR + 1, WC = 2 * BC + 1, LDE = CIN + 8; /* window, LDS pixel stride (halfs) */
    constexpr int NPX = BR * BC, TT = NPX / 16, TPR = BC / 16;
    constexpr int RTALL = COUT / 16, RT = RTALL / 4, CPT = CIN / 32, KS = 9 * CPT;
    constexpr int LDO = COUT + 8;
    static_assert(BC % 16 == 0 && RTALL % 4 == 0 && CIN % 32 == 0 && DW >= 1 && DW <= KS, "window stage shape");
    static_assert(WR * WC * LDE >= NPX * LDO, "the output tile fits where the window was");
    __shared__ __attribute__((aligned(16))) f16 win[WR * WC * LDE];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int iw = a.in_w, ih = a.in_h, ow = a.out_w, oh = a.out_h;
    const int bxn = (ow + BC - 1) / BC;
    const int blk = codec_block<BAND>();
    const int oy0 = (blk / bxn) * BR, ox0 = (blk % bxn) * BC;
    const int wy0 = 2 * oy0 - 1, wx0 = 2 * ox0 - 1;
    codec_map_window<CIN, WR, WC, LDE, 256>(
        MapSrc(a.in + (int64_t)blockIdx.y * a.in_frame, (uint32_t)(a.in_frame * 2)), iw, ih, wy0, wx0, win);
    __syncthreads();
    const int rt0 = wave * RT;
    f4 acc[RT][TT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int ch = 16 * (rt0 + r) + 4 * g;
        const f4 bb = {a.b[ch], a.b[ch + 1], a.b[ch + 2], a.b[ch + 3]};
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = bb;
    }
    /* this lane's window pixel for tap 0 of each tile (byte offsets) */
    uint32_t boff[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const int ly = t / TPR, lx = 16 * (t % TPR) + l16;
        boff[t] = (uint32_t)(((2 * ly * WC + 2 * lx) * LDE + 8 * g) * 2);
    }
    const unsigned char* wb = reinterpret_cast<const unsigned char*>(win);
    auto bload = [&](int ks, int t) {
        const int tap = ks / CPT, c = ks % CPT;
        return *reinterpret_cast<const h8*>(wb + boff[t] + (((tap / 3) * WC + tap % 3) * LDE + 32 * c) * 2);
    };
    const FragSrc wsrc(a.w, (unsigned)(RTALL * KS * 1024));
    h8 wq[DW][RT];
#pragma unroll
    for (int d = 0; d < DW; ++d)
#pragma unroll
        for (int r = 0; r < RT; ++r) wq[d][r] = wsrc.load((rt0 + r) * KS + d, lane * 16);
    h8 bc[TT], bn[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) bc[t] = bload(0, t);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        if (ks + 1 < KS) {
#pragma unroll
            for (int t = 0; t < TT; ++t) bn[t] = bload(ks + 1, t);
        }
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int t = 0; t < TT; ++t) acc[r][t] = mfma_16x16x32(wq[ks % DW][r], bc[t], acc[r][t]);
        if (ks + DW < KS) {
#pragma unroll
            for (int r = 0; r < RT; ++r) wq[ks % DW][r] = wsrc.load((rt0 + r) * KS + ks + DW, lane * 16);
        }
        if (ks + 1 < KS) {
#pragma unroll
            for (int t = 0; t < TT; ++t) bc[t] = bn[t];
        }
        sched_fence();
    }
    __syncthreads(); /* every wave is done reading the window */
    f16* otile = win;
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            f4 v = acc[r][t];
            /* max(r16(v), 0) == r16(max(v, 0)): fp16 rounding is monotonic */
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = fmaxf(v[i], 0.f);
            *reinterpret_cast<h4*>(otile + (16 * t + l16) * LDO + 16 * (rt0 + r) + 4 * g) = cvt_h4(v);
        }
    __syncthreads();
    uint16_t* out = a.out + (int64_t)blockIdx.y * a.out_frame;
    codec_store_block<NPX, COUT / 8, 256>([&](int pl) { return otile + pl * LDO; }, [&](int pl) {
        const int y = oy0 + pl / BC, x = ox0 + pl % BC;
        return y < oh && x < ow ? out + ((int64_t)y * ow + x) * COUT : nullptr;
    });
}

/* A stride-2 conv3x3's taps read from an LDS copy of the input region under
 * an output block at (y0, x0): output pixel (y, x) and tap (ky, kx) read
 * region pixel (2 (y - y0) + ky, 2 (x - x0) + kx), EC pixels a region row,
 * LDE halfs a pixel, zeros where the region leaves the map; k = tap * CIN +
 * ic as SrcConvNHWC. For pixels past the map the offsets stay in the region. */
template <int CIN, int EC, int LDE>
struct SrcRegionLds {
    static constexpr int KS = 9 * CIN / 32, CPT = CIN / 32;
    const f16* lds;
    int y0, x0;
    struct Pix {
        uint32_t off[9];
    };
    __device__ __forceinline__ Pix prep(const CodecPix& p, int g) const {
        Pix q;
        const int r0 = 2 * (p.y - y0), c0 = 2 * (p.x - x0);
#pragma unroll
        for (int tap = 0; tap < 9; ++tap)
            q.off[tap] = (uint32_t)((((r0 + tap / 3) * EC + c0 + tap % 3) * LDE + 8 * g) * 2);
        return q;
    }
    /* k-step i KSP + j (i compile-time, j < KSP wave-uniform) */
    template <int KSP>
    __device__ __forceinline__ h8 load(int i, int j, const Pix& q) const {
        static_assert(CPT % KSP == 0, "a split's k-steps stay within one tap");
        return *reinterpret_cast<const h8*>(reinterpret_cast<const unsigned char*>(lds) + q.off[i * KSP / CPT] +
                                            (((i * KSP) % CPT + j) * 64));
    }
};

/* enc0 + enc1 in one launch (prism_encode and the end-to-end frame; the stage
 * calls keep them apart). A workgroup takes a BR x BC block of enc1 outputs at
 * r1 (y1, x1) (4 x 32: of 4 x 16 and 2 x 32 at 960 x 540 the fastest). Its
 * stride-2 taps need e0 rows 2 y1 - 1 .. 2 y1 + 2 BR - 1 and columns
 * 2 x1 - 1 .. 2 x1 + 2 BC - 1, a (2 BR + 1) x (2 BC + 1) region (9 x 65): the
 * workgroup copies the frame under it (2 more rows and columns, 16 halfs a
 * pixel as in enc0) into LDS,
 * computes enc0 for the region (the same fragments, tap order, rounding and
 * ReLU as prism_codec_enc0; region pixels 16 to a tile in row-major order,
 * one halo row and column recomputed by the neighbours) into a second LDS
 * array, writes its own 2 BR x 2 BC e0 pixels to the e0 map (the decoder's skip),
 * and runs enc1 with its B fragments read from that array (as
 * prism_codec_enc1: k = tap * 32 + ic, the same fragments and order).
 * Outputs equal the two separate launches bit for bit. Grid: x =
 * ceil(w1/BC) * ceil(h1/BR) blocks in XCD bands, y = frames. a0, a1: enc0's
 * and enc1's arguments (a1.in unused). */
template <int BR, int BC>
__device__ __forceinline__ void codec_enc01(const CodecArgs& a0, const CodecArgs& a1) {
    constexpr int CH = 9, CP = 16, KS0 = 5;
    static_assert((BR == 2 || BR == 4) && BC % 16 == 0 && BR * BC % 64 == 0, "block of whole tiles per wave");
    constexpr int NPX = BR * BC, TT = NPX / 64, TPR = BC / 16; /* block pixels, tiles per wave, tiles per row */
    constexpr int ER = 2 * BR + 1, EC = 2 * BC + 1, LDE = 40; /* the e0 region, 32 channels a pixel */
    using Src = SrcRegionLds<32, EC, LDE>;
    constexpr int FR = ER + 2, FC = EC + 2;                        /* the frame window */
    constexpr int NREG = ER * EC, NT0 = (NREG + 15) / 16;          /* region pixels, their tiles */
    constexpr int LDO = 64 + 8;                                    /* e1 staging row (halfs) */
    __shared__ __attribute__((aligned(16))) f16 s_in[FR * FC * CP]; /* frame window, then e1 staging */
    __shared__ __attribute__((aligned(16))) f16 e0s[NREG * LDE];
    static_assert(FR * FC * CP >= NPX * LDO, "the e1 tile fits where the frame window was");
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int W0 = a0.out_w, H0 = a0.out_h, W1 = a1.out_w, H1 = a1.out_h;
    const int bxn = (W1 + BC - 1) / BC;
    const int blk = codec_block<true>();
    const int y1 = (blk / bxn) * BR, x1 = (blk % bxn) * BC; /* r1 block origin */
    const int ey0 = 2 * y1 - 1, ex0 = 2 * x1 - 1;          /* e0 region origin */
    /* ---- the frame window (origin ey0 - 1, ex0 - 1), 16 halfs a pixel */
    codec_frame_window<FR, FC>(reinterpret_cast<const f16*>(a0.in) + (int64_t)blockIdx.y * a0.in_frame, W0, H0,
                               ey0 - 1, ex0 - 1, s_in);
    __syncthreads();
    /* ---- enc0 for the region; wave w takes region tiles w, w + 4, ... */
    {
        const FragSrc wsrc(a0.w, 2u * KS0 * 1024u);
        h8 wf[2][KS0];
#pragma unroll
        for (int ks = 0; ks < KS0; ++ks) {
            wf[0][ks] = wsrc.load(0 * KS0 + ks, lane * 16);
            wf[1][ks] = wsrc.load(1 * KS0 + ks, lane * 16);
        }
        f4 bias[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int ch = 16 * r + 4 * g;
            bias[r] = f4{a0.b[ch], a0.b[ch + 1], a0.b[ch + 2], a0.b[ch + 3]};
        }
        uint16_t* e0map = a0.out + (int64_t)blockIdx.y * a0.out_frame;
        for (int tile = wave; tile < NT0; tile += 4) { /* uniform over the wave */
            const int p = min(16 * tile + l16, NREG - 1); /* past the region: a copy of its last pixel */
            const int er = p / EC, ec = p - er * EC;
            f4 acc[2] = {bias[0], bias[1]};
#pragma unroll
            for (int ks = 0; ks < KS0; ++ks) {
                /* k = 32 ks + 8 g + j = tap * 16 + 8 (g & 1) + j; tap 9 is padding (zero) */
                const int tap = 2 * ks + (g >> 1), tc = tap < CH ? tap : CH - 1;
                const int ky = tc / 3, kx = tc - 3 * ky;
                h8 b = *reinterpret_cast<const h8*>(s_in + ((er + ky) * FC + ec + kx) * CP + 8 * (g & 1));
                if (tap >= CH) b = h8{};
                acc[0] = mfma_16x16x32(wf[0][ks], b, acc[0]);
                acc[1] = mfma_16x16x32(wf[1][ks], b, acc[1]);
            }
            const int gy = ey0 + er, gx = ex0 + ec;
            const bool inmap = gy >= 0 && gy < H0 && gx >= 0 && gx < W0;
            const bool mine = inmap && er >= 1 && ec >= 1 && 16 * tile + l16 < NREG; /* this block's e0 pixels */
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                f4 v = acc[r];
                /* max(r16(v), 0) == r16(max(v, 0)): fp16 rounding is monotonic */
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = fmaxf(v[i], 0.f);
                const h4 hv = cvt_h4(v);
                /* enc1's zero padding where the region leaves the map */
                *reinterpret_cast<h4*>(e0s + p * LDE + 16 * r + 4 * g) = inmap ? hv : h4{};
                if (mine) *reinterpret_cast<h4*>(e0map + ((int64_t)gy * W0 + gx) * 32 + 16 * r + 4 * g) = hv;
            }
        }
    }
    __syncthreads();
    /* ---- enc1 for the block: wave w takes its TT 16-pixel tiles, row-major */
    CodecPix px[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const int tile = wave * TT + t;
        px[t].y = y1 + tile / TPR;
        px[t].x = x1 + 16 * (tile % TPR) + l16;
        px[t].valid = px[t].y < H1 && px[t].x < W1;
    }
    const Src src{e0s, y1, x1};
    f4 acc[4][TT];
    codec_gemm<Src, 4, 4, TT>(src, a1.w, a1.b, px, g, lane, 0, acc);
    f16* otile = s_in; /* the frame window is dead since the barrier above */
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            f4 v = acc[r][t];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = fmaxf(v[i], 0.f);
            *reinterpret_cast<h4*>(otile + (16 * (wave * TT + t) + l16) * LDO + 16 * r + 4 * g) = cvt_h4(v);
        }
    __syncthreads();
    uint16_t* e1map = a1.out + (int64_t)blockIdx.y * a1.out_frame;
    codec_store_block<NPX, 8, 256>([&](int pl) { return otile + pl * LDO; }, [&](int pl) {
        const int Y = y1 + pl / BC, X = x1 + pl % BC;
        return Y < H1 && X < W1 ? e1map + ((int64_t)Y * W1 + X) * 64 : nullptr;
    });
}

/* enc2 + enc3 in one launch (prism_encode and the end-to-end frame; the stage
 * calls keep them apart), 8 waves. A workgroup takes a BR x BC block of enc3
 * outputs (32 pixels) at r3 (y3, x3). enc3's stride-2 taps need e2 rows
 * 2 y3 - 1 .. 2 y3 + 2 BR - 1 and columns 2 x3 - 1 .. 2 x3 + 2 BC - 1, a
 * (2 BR + 1) x (2 BC + 1) region, whose own taps need a (4 BR + 3) x
 * (4 BC + 3) window of e1. The workgroup copies that e1 window into LDS,
 * computes enc2 for the region into a second LDS array with each wave taking
 * one of enc2's 8 output row tiles over all the region's pixels (as
 * prism_codec_enc2: the same fragments, k order, rounding and ReLU; zeros
 * where the region leaves the map, which is enc3's padding), writes its own
 * 2 BR x 2 BC e2 pixels to the e2 map (the decoder's skip) as whole pixel
 * rows, and runs enc3 from the region as prism_codec_enc3 does: its
 * reduction split over KSP = 4 waves (two pixel groups of one 16-pixel tile
 * each), partials summed in wave order. Outputs equal the two separate
 * launches bit for bit. Grid: x = ceil(w3/BC) * ceil(h3/BR) blocks, y =
 * frames. a2, a3: enc2's and enc3's arguments (a3.in unused). */
template <int BR, int BC, bool BAND>
__device__ __forceinline__ void codec_enc23(const CodecArgs& a2, const CodecArgs& a3) {
    constexpr int C1 = 64, C2 = 128, C3 = 128, NW = 8, KSP = 4;
    constexpr int ER = 2 * BR + 1, EC = 2 * BC + 1;          /* the e2 region */
    constexpr int WR = 2 * ER + 1, WC = 2 * EC + 1;          /* the e1 window */
    constexpr int L1 = C1 + 8, L2 = C2 + 8, LDO = C3 + 8;    /* LDS pixel strides (halfs) */
    constexpr int NREG = ER * EC, NT2 = (NREG + 15) / 16;    /* region pixels, their tiles */
    constexpr int NPX = BR * BC, TT3 = 1;                    /* enc3 block: 2 groups x 1 tile */
    constexpr int RT3 = C3 / 16, NO = RT3 - RT3 / KSP;
    constexpr int CPT2 = C1 / 32, KS2 = 9 * CPT2, RTALL2 = C2 / 16, DW = 3;
    static_assert(NPX == 16 * TT3 * NW / KSP && RTALL2 == NW, "8 waves: one enc2 row tile each, 2 x 4 for enc3");
    static_assert(NW * NO * TT3 * 64 * 16 + NPX * LDO * 2 <= WR * WC * L1 * 2,
                  "enc3's partials and output tile fit where the e1 window was");
    __shared__ __attribute__((aligned(16))) f16 win[WR * WC * L1]; /* e1 window; then partials + e3 tile */
    __shared__ __attribute__((aligned(16))) f16 e2s[NREG * L2];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int W1 = a2.in_w, H1 = a2.in_h, W2 = a2.out_w, H2 = a2.out_h, W3 = a3.out_w, H3 = a3.out_h;
    const int bxn = (W3 + BC - 1) / BC;
    const int blk = codec_block<BAND>();
    const int y3 = (blk / bxn) * BR, x3 = (blk % bxn) * BC; /* r3 block origin */
    const int ey0 = 2 * y3 - 1, ex0 = 2 * x3 - 1;          /* e2 region origin */
    const int wy0 = 2 * ey0 - 1, wx0 = 2 * ex0 - 1;        /* e1 window origin */
    /* ---- the e1 window */
    codec_map_window<C1, WR, WC, L1, 64 * NW>(
        MapSrc(a2.in + (int64_t)blockIdx.y * a2.in_frame, (uint32_t)(a2.in_frame * 2)), W1, H1, wy0, wx0, win);
    __syncthreads();
    /* ---- enc2 for the region: wave w takes row tile w over all NT2 tiles */
    {
        f4 acc[NT2];
        {
            const int ch = 16 * wave + 4 * g;
            const f4 bb = {a2.b[ch], a2.b[ch + 1], a2.b[ch + 2], a2.b[ch + 3]};
#pragma unroll
            for (int t = 0; t < NT2; ++t) acc[t] = bb;
        }
        uint32_t boff[NT2]; /* this lane's window pixel for tap 0 of each tile (bytes) */
#pragma unroll
        for (int t = 0; t < NT2; ++t) {
            const int p = min(16 * t + l16, NREG - 1); /* past the region: a copy of its last pixel */
            const int er = p / EC, ec = p - er * EC;
            boff[t] = (uint32_t)(((2 * er * WC + 2 * ec) * L1 + 8 * g) * 2);
        }
        const unsigned char* wb = reinterpret_cast<const unsigned char*>(win);
        auto bload = [&](int ks, int t) {
            const int tap = ks / CPT2, c = ks % CPT2;
            return *reinterpret_cast<const h8*>(wb + boff[t] + (((tap / 3) * WC + tap % 3) * L1 + 32 * c) * 2);
        };
        const FragSrc wsrc(a2.w, (unsigned)(RTALL2 * KS2 * 1024));
        h8 wq[DW];
#pragma unroll
        for (int d = 0; d < DW; ++d) wq[d] = wsrc.load(wave * KS2 + d, lane * 16);
        h8 bc[NT2], bn[NT2];
#pragma unroll
        for (int t = 0; t < NT2; ++t) bc[t] = bload(0, t);
#pragma unroll
        for (int ks = 0; ks < KS2; ++ks) {
            if (ks + 1 < KS2) {
#pragma unroll
                for (int t = 0; t < NT2; ++t) bn[t] = bload(ks + 1, t);
            }
#pragma unroll
            for (int t = 0; t < NT2; ++t) acc[t] = mfma_16x16x32(wq[ks % DW], bc[t], acc[t]);
            if (ks + DW < KS2) wq[ks % DW] = wsrc.load(wave * KS2 + ks + DW, lane * 16);
            if (ks + 1 < KS2) {
#pragma unroll
                for (int t = 0; t < NT2; ++t) bc[t] = bn[t];
            }
            sched_fence();
        }
#pragma unroll
        for (int t = 0; t < NT2; ++t) {
            const int p = 16 * t + l16;
            if (p < NREG) {
                const int er = p / EC, ec = p - er * EC;
                const int gy = ey0 + er, gx = ex0 + ec;
                const bool inmap = gy >= 0 && gy < H2 && gx >= 0 && gx < W2;
                f4 v = acc[t];
                /* max(r16(v), 0) == r16(max(v, 0)): fp16 rounding is monotonic */
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = fmaxf(v[i], 0.f);
                *reinterpret_cast<h4*>(e2s + p * L2 + 16 * wave + 4 * g) = inmap ? cvt_h4(v) : h4{};
            }
        }
    }
    __syncthreads(); /* the region is complete; the e1 window is dead */
    /* ---- this block's e2 pixels (region rows and columns 1 .. 2 BR, 2 BC) to the e2 map */
    {
        uint16_t* e2 = a2.out + (int64_t)blockIdx.y * a2.out_frame;
        codec_store_block<4 * NPX, C2 / 8, 64 * NW>(
            [&](int pl) { return e2s + ((1 + pl / (2 * BC)) * EC + 1 + pl % (2 * BC)) * L2; }, [&](int pl) {
                const int gy = ey0 + 1 + pl / (2 * BC), gx = ex0 + 1 + pl % (2 * BC);
                return gy < H2 && gx < W2 ? e2 + ((int64_t)gy * W2 + gx) * C2 : nullptr;
            });
    }
    /* ---- enc3 for the block: pixel group wave / KSP (16 pixels, row-major
       over the block), k-steps kq, kq + KSP, ... for wave position kq */
    CodecPix px[TT3];
    {
        const int pl = 16 * (wave / KSP) + l16;
        px[0].y = y3 + pl / BC;
        px[0].x = x3 + pl % BC;
        px[0].valid = px[0].y < H3 && px[0].x < W3;
    }
    using Src = SrcRegionLds<C2, EC, L2>;
    const Src src{e2s, y3, x3};
    f4 acc[RT3][TT3];
    codec_gemm<Src, RT3, RT3, TT3, KSP>(src, a3.w, a3.b, px, g, lane, 0, acc, wave % KSP);
    f4* part = reinterpret_cast<f4*>(win);
    f16* otile = win + NW * NO * TT3 * 64 * 8;
    codec_ksplit_reduce<RT3, TT3, KSP, LDO>(acc, part, otile, wave, lane, l16, g);
    __syncthreads();
    uint16_t* e3 = a3.out + (int64_t)blockIdx.y * a3.out_frame;
    codec_store_block<NPX, C3 / 8, 64 * NW>([&](int pl) { return otile + pl * LDO; }, [&](int pl) {
        const int y = y3 + pl / BC, x = x3 + pl % BC;
        return y < H3 && x < W3 ? e3 + ((int64_t)y * W3 + x) * C3 : nullptr;
    });
}

#define CODEC_FRAME(p, n) ((p) + (int64_t)blockIdx.y * (n))
#define CODEC_IN_MAP MapSrc(CODEC_FRAME(a.in, a.in_frame), (uint32_t)(a.in_frame * 2))
#define CODEC_SKIP_MAP MapSrc(CODEC_FRAME(a.skip, a.skip_frame), (uint32_t)(a.skip_frame * 2))

extern "C" __global__ void __launch_bounds__(256) prism_codec_enc0(CodecArgs a) { codec_enc0_body(a); }
extern "C" __global__ void __launch_bounds__(256) prism_codec_enc01(CodecArgs a0, CodecArgs a1) {
    codec_enc01<CODEC_ENC01_ROWS, CODEC_ENC01_COLS>(a0, a1);
}
extern "C" __global__ void __launch_bounds__(512) prism_codec_enc23(CodecArgs a2, CodecArgs a3) {
    codec_enc23<CODEC_ENC23_ROWS, CODEC_ENC23_COLS, CODEC_ENC23_BAND>(a2, a3);
}
extern "C" __global__ void __launch_bounds__(256) prism_codec_enc1(CodecArgs a) {
    codec_stage_any<SrcConvNHWC<32, 2>, 64, CODEC_TT_ENC1, CODEC_RS_ENC1, CODEC_KSP_ENC1, true>(a, SrcConvNHWC<32, 2>{CODEC_IN_MAP, a.in_w, a.in_h});
}
extern "C" __global__ void __launch_bounds__(256) prism_codec_enc2(CodecArgs a) {
    codec_conv_window<64, 128, CODEC_WIN_ROWS_ENC2, CODEC_WIN_COLS_ENC2, CODEC_WIN_DW_ENC2, true>(a);
}
extern "C" __global__ void __launch_bounds__(256) prism_codec_enc3(CodecArgs a) {
    codec_stage_any<SrcConvNHWC<128, 2>, 128, CODEC_TT_ENC3, CODEC_RS_ENC3, CODEC_KSP_ENC3, false>(a, SrcConvNHWC<128, 2>{CODEC_IN_MAP, a.in_w, a.in_h});
}
extern "C" __global__ void __launch_bounds__(256) prism_codec_dec3(CodecArgs a) {
    codec_stage_any<SrcDec<128, 128>, 128, CODEC_TT_DEC3, CODEC_RS_DEC3, CODEC_KSP_DEC3, false>(
        a, SrcDec<128, 128>{CODEC_IN_MAP, CODEC_SKIP_MAP, a.in_w, a.in_h, a.out_w});
}
extern "C" __global__ void __launch_bounds__(256) prism_codec_dec2(CodecArgs a) {
    codec_stage_any<SrcDec<128, 64>, 64, CODEC_TT_DEC2, CODEC_RS_DEC2, CODEC_KSP_DEC2, true>(
        a, SrcDec<128, 64>{CODEC_IN_MAP, CODEC_SKIP_MAP, a.in_w, a.in_h, a.out_w});
}
extern "C" __global__ void __launch_bounds__(256) prism_codec_dec1_out(CodecArgs a) { codec_dec_out<CODEC_TT_DEC1>(a); }
extern "C" __global__ void __launch_bounds__(256) prism_codec_dec21_out(CodecArgs a2, CodecArgs a1) {
    codec_dec21_out(a2, a1);
}
#undef CODEC_FRAME
#undef CODEC_IN_MAP
#undef CODEC_SKIP_MAP
