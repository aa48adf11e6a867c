// Repacking that runs ahead of the fused forward/backward, as one launch:
//
// input : NCHW input -> channels-last xt [B][H*W][G*Cgp] with zeroed padding
//         channels, so a bilinear corner is one contiguous channel vector
//         (16-byte loads) instead of C scattered scalars.  The reference
//         samples NCHW directly, one scalar per thread (com.cu:151-195).
// weight: [Cout][C/WG][kh][kw] -> MFMA fragment order of W' [Mp][Kp] (or of
//         its transpose) with K ordered (tap, group, channel) and zero padding,
//         plus the chunk table.  With WG weight groups W' is block diagonal:
//         row m holds its group's C/WG channels and zeros for all others, so
//         the GEMMs need no notion of groups.
//
// Blocks [0, nw) pack 256 16-byte pieces of the weight each; blocks
// [nw, nw + nin) transpose 64 pixels x CT channels of the input each (CT*esz
// = 128 bytes, one channel chunk of a pixel); the rest clear accumulators.
// The halves are independent, so the (small, latency bound) weight packing,
// dispatched first, overlaps the (bandwidth bound) input transpose.
#include "dcn2_common.h"
#include "dcn2_kernels.h"
#include "../../include/dcnv2_amd.h"

namespace dcn2 {

struct PackParams {
    const void *in, *w;
    void *xt, *wp;
    int4 *tab;
    int B, C, HW, Cg, Cgp, cs;     // input geometry
    int pxt, cht, nin;             // pixel tiles, channel tiles per image, input blocks
    int in_vec;                    // HW % E == 0 and 16-byte aligned input: vector loads
    int Cout, KK, kw, dh, dw, G;   // weight geometry
    int Cw, mpg;                   // channels and output channels per weight group
    int kc, kstep, kpl, Mp, Kp;    // MFMA packing
    int transpose;                 // 0: forward A fragments, 1: backward W'^T fragments
    int nhwc;                      // input is channels-last [B][HW][C]
    int nw;                        // weight blocks
    float4 *clr[kClearBufs];       // buffers to zero, 16-byte pieces each
    long clr_n4[kClearBufs];
    int clr_blk[kClearBufs + 1];   // first clearing block of each buffer (prefix sums)
};
constexpr int kClearPieces = 1024;  // 16-byte pieces zeroed per clearing block

// Pixels of one input block (64: measured alone at c1, 7 TB/s, against 6.3 TB/s
// for 128; inside the forward step the two sizes measure the same).
constexpr int kPackPx = 64;

// Channels-last input [B][HW][C] -> xt [B][HW][cs]: the same tile of kPackPx
// pixels x CT padded channels, one element per thread and step (consecutive
// threads take consecutive channels of a pixel, so both sides are contiguous).
// Only used when the padding makes xt differ from the input; otherwise the
// kernels read the input in place.
template <typename T>
__device__ __forceinline__ void pack_input_block_nhwc(const PackParams &p, int blk) {
    constexpr int CT = 128 / sizeof(T);
    const T *__restrict__ in = (const T *)p.in;
    T *__restrict__ xt = (T *)p.xt;
    const int pt = blk % p.pxt, ct = (blk / p.pxt) % p.cht, b = blk / (p.pxt * p.cht);
    const int px0 = pt * kPackPx, cp0 = ct * CT;
#pragma unroll 8
    for (int k = 0; k < kPackPx * CT / 256; ++k) {
        const int idx = threadIdx.x + k * 256;
        const int pl = idx / CT, cl = idx - pl * CT;
        const int px = px0 + pl, cp = cp0 + cl;
        if (px >= p.HW) continue;
        const int g = cp / p.Cgp, ci = cp - g * p.Cgp;
        T v = (T)0.0f;
        if (ci < p.Cg) v = in[((size_t)b * p.HW + px) * p.C + g * p.Cg + ci];
        xt[((size_t)b * p.HW + px) * p.cs + cp] = v;
    }
}

// Input transpose: kPackPx pixels x CT padded channels per block, 256 threads.
template <typename T>
__device__ __forceinline__ void pack_input_block(const PackParams &p, int blk) {
    constexpr int E = 16 / sizeof(T);     // elements per 16-byte vector
    constexpr int CT = 128 / sizeof(T);   // channels per block (128 bytes of a pixel)
    constexpr int PX = kPackPx;
    // LDS tile [channel][pixel], the 16-byte blocks of channel row c XOR-permuted
    // by (c / E) % 8: the transposed reads (the E channels of one pixel, for 8
    // consecutive channel blocks across lanes) then hit 8 distinct banks.
    constexpr int LDP = PX;               // LDS pitch (elements) of one channel row
    __shared__ __attribute__((aligned(16))) T tile[CT][LDP];
    const T *__restrict__ in = (const T *)p.in;
    T *__restrict__ xt = (T *)p.xt;
    const int tid = threadIdx.x;
    const int pt = blk % p.pxt, ct = (blk / p.pxt) % p.cht, b = blk / (p.pxt * p.cht);
    const int px0 = pt * PX, cp0 = ct * CT;

    // load: CT channel rows of PX pixels, E pixels per lane
    constexpr int LPR = PX / E;  // lanes per channel row
#pragma unroll
    for (int k = 0; k < CT * LPR / 256; ++k) {
        const int idx = tid + k * 256;
        const int cl = idx / LPR, po = (idx - cl * LPR) * E;
        const int cp = cp0 + cl, g = cp / p.Cgp, ci = cp - g * p.Cgp;
        const bool live = ci < p.Cg;
        const T *src = in + ((size_t)b * p.C + g * p.Cg + (live ? ci : 0)) * p.HW + px0 + po;
        if (p.in_vec) {
            uint4 v = make_uint4(0, 0, 0, 0);
            if (live && px0 + po < p.HW) v = *reinterpret_cast<const uint4 *>(src);
            *reinterpret_cast<uint4 *>(&tile[cl][((po / E) ^ ((cl / E) & 7)) * E]) = v;
        } else {
#pragma unroll
            for (int e = 0; e < E; ++e)
                tile[cl][((po / E) ^ ((cl / E) & 7)) * E + e] = (live && px0 + po + e < p.HW) ? src[e] : (T)0.0f;
        }
    }
    __syncthreads();
    // store: one 16-byte run of E channels of one pixel per lane
    constexpr int VPP = CT / E;  // vectors per pixel
#pragma unroll
    for (int k = 0; k < PX * VPP / 256; ++k) {
        const int idx = tid + k * 256;
        const int pl = idx / VPP, cg = (idx - pl * VPP) * E;
        if (px0 + pl >= p.HW) continue;
        T v[E];
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = tile[cg + e][((pl / E) ^ (((cg + e) / E) & 7)) * E + pl % E];
        *reinterpret_cast<uint4 *>(xt + ((size_t)b * p.HW + px0 + pl) * p.cs + cp0 + cg) =
            __builtin_bit_cast(uint4, v);
    }
}

// One thread per 16-byte piece (EPT = 16/esz consecutive elements) of the
// packed weight.  transpose 0 (forward): MFMA A-fragment order,
// dst[((rb*nch + ch)*nks + ks)*64 + lane][e] holds
// W'[32*rb + lane%32][ch*kc + ks*kstep + (lane/32)*kpl + e], so one wave's
// fragment load is one contiguous run; transpose 1 (backward): the same for
// W'^T (rows k, reduction m): dst[((kb*(Mp/kstep) + ms)*64 + lane)][e] holds
// W'[ms*kstep + (lane/32)*kpl + e][32*kb + lane%32].  For 2-byte types a
// piece is the kpl = 8 elements e of one lane; for fp32 (kpl = 1) it is
// 4 consecutive lanes.  All index math is 32-bit (the host bounds Mp*Kp
// below 2^31).
// The first nch threads also write the chunk table: for chunk ch of the K
// order (tap, group, channel chunk of kc channels) tab[ch] = {offset/mask
// plane g*KK + tap, row term ki*dh, column term kj*dw, channel base
// g*Cgp + cc*kc}; the sampling kernels read it with scalar loads instead of
// dividing the chunk index every step.
template <typename T>
__device__ __forceinline__ void pack_weight_block(const PackParams &p, int blk) {
    constexpr int EPT = 16 / sizeof(T);
    const T *__restrict__ w = (const T *)p.w;
    T *__restrict__ dst = (T *)p.wp;
    const int t = blk * 256 + threadIdx.x;
    const int nch = p.Kp / p.kc;
    if (p.tab && t < nch) {
        const int cpg = p.Cgp / p.kc;
        const int tg = t / cpg, cc = t - tg * cpg;
        const int tap = tg / p.G, g = tg - tap * p.G;
        const int ki = tap / p.kw, kj = tap - ki * p.kw;
        p.tab[t] = make_int4(g * p.KK + tap, ki * p.dh, kj * p.dw, g * p.Cgp + cc * p.kc);
    }
    const int idx0 = t * EPT;
    if (idx0 >= p.Mp * p.Kp) return;
    const int kpl = p.kpl, kstep = p.kstep;
    // fragment coordinates of element idx0: e0, lane0 and the fragment index
    const int e0 = idx0 % kpl;
    int r = idx0 / kpl;
    const int lane0 = r % 64;
    r /= 64;
    int a = 0, bq = 0;  // transpose 0: (ks, ch, rb); 1: (ms, kb)
    int ks = 0, ch = 0;
    if (p.transpose) {
        const int nms = p.Mp / kstep;
        a = r % nms;  // ms
        bq = r / nms; // kb
    } else {
        const int nks = p.kc / kstep;
        ks = r % nks;
        r /= nks;
        ch = r % nch;
        bq = r / nch; // rb
    }
    // Across the EPT elements of a piece one coordinate steps by one and the
    // other is fixed: for 2-byte types (kpl = 8) the K index (the channel c,
    // within one tap and group: a piece never crosses a KC-channel chunk) in
    // the forward layout and the row m in the transposed one; for fp32
    // (kpl = 1, consecutive lanes) the row m in the forward layout and the K
    // index in the transposed one.  So the divisions run once per piece.
    const bool step_k = (kpl > 1) != (p.transpose != 0);
    int m0, k0;
    if (p.transpose) {
        k0 = bq * 32 + (lane0 & 31);
        m0 = a * kstep + (lane0 >> 5) * kpl + e0;
    } else {
        m0 = bq * 32 + (lane0 & 31);
        k0 = ch * p.kc + ks * kstep + (lane0 >> 5) * kpl + e0;
    }
    const int gc = p.G * p.Cgp;
    const int tap = k0 / gc, rr = k0 - tap * gc;
    const int g = rr / p.Cgp, c0 = rr - g * p.Cgp;
    T v[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int m = step_k ? m0 : m0 + j;
        const int c = step_k ? c0 + j : c0;
        // input channel g*Cg + c, as channel cl of row m's weight group
        const int cl = g * p.Cg + c - (m / p.mpg) * p.Cw;
        v[j] = (m < p.Cout && c < p.Cg && (unsigned)cl < (unsigned)p.Cw)
                   ? w[((size_t)m * p.Cw + cl) * p.KK + tap]
                   : (T)0.0f;
    }
    *reinterpret_cast<uint4 *>(dst + idx0) = __builtin_bit_cast(uint4, v);
}

template <typename T>
__global__ __launch_bounds__(256) void pack_kernel(const PackParams p) {
    // weight blocks first: they are latency bound, so they are dispatched
    // ahead of (and overlap) the bandwidth-bound input transpose
    const int blk = blockIdx.x;
    if (blk < p.nw) {
        pack_weight_block<T>(p, blk);
    } else if (blk < p.nw + p.nin) {
        if (p.nhwc)
            pack_input_block_nhwc<T>(p, blk - p.nw);
        else
            pack_input_block<T>(p, blk - p.nw);
    } else {
        // zero kClearPieces 16-byte pieces of one of the clear-list buffers
        const int cb = blk - p.nin - p.nw;
        int i = 0;
#pragma unroll
        for (int k = 1; k < kClearBufs; ++k) i = cb >= p.clr_blk[k] ? k : i;
        const long base = (long)(cb - p.clr_blk[i]) * kClearPieces;
        for (int k = threadIdx.x; k < kClearPieces; k += 256)
            if (base + k < p.clr_n4[i]) p.clr[i][base + k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
}

template <typename T>
static hipError_t pack_t(const Geo &g, const void *input, void *xt, const void *weight,
                         void *wp, void *tab, bool transpose, hipStream_t s, const ClearList *clear) {
    constexpr int E = 16 / sizeof(T), CT = 128 / sizeof(T);
    PackParams p;
    p.in = input;
    p.w = weight;
    p.xt = xt;
    p.wp = wp;
    p.tab = (int4 *)tab;
    p.B = g.B;
    p.C = g.C;
    p.HW = g.H * g.W;
    p.Cg = g.Cg;
    p.Cgp = g.Cgp;
    p.cs = g.cs;
    p.pxt = ceil_div(p.HW, kPackPx);
    p.cht = g.cs / CT;  // cs is a multiple of the chunk KC, and KC == CT
    p.nin = input ? g.B * p.pxt * p.cht : 0;
    p.in_vec = (p.HW % E == 0) && (((uintptr_t)input & 15) == 0);
    p.Cout = g.Cout;
    p.KK = g.KK;
    p.kw = g.kw;
    p.dh = g.dh;
    p.dw = g.dw;
    p.G = g.G;
    p.Cw = g.Cw;
    p.mpg = g.Cout / g.WG;
    p.kc = g.KC;
    p.kstep = g.dtype == DCN2_F32 ? 2 : 16;
    p.kpl = g.dtype == DCN2_F32 ? 1 : 8;
    p.Mp = g.Mp;
    p.Kp = g.Kp;
    p.transpose = transpose ? 1 : 0;
    p.nhwc = g.nhwc;
    // one thread per 16-byte piece of the packed weight (Mp*Kp is a multiple of
    // 16/esz); none when weight is null (a later slice of the backward, whose
    // packed weight and table the first slice wrote)
    const long nw = weight ? ((long)g.Mp * g.Kp / E + 255) / 256 : 0;
    p.nw = (int)nw;
    p.clr_blk[0] = 0;
    for (int i = 0; i < kClearBufs; ++i) {
        const size_t n = clear ? clear->n[i] : 0;
        p.clr[i] = n ? (float4 *)clear->p[i] : nullptr;
        p.clr_n4[i] = (long)((n + 3) / 4);
        p.clr_blk[i + 1] = p.clr_blk[i] + (int)((p.clr_n4[i] + kClearPieces - 1) / kClearPieces);
    }
    const long blocks = p.nin + nw + p.clr_blk[kClearBufs];
    pack_kernel<T><<<(unsigned)blocks, 256, 0, s>>>(p);
    return hipGetLastError();
}

hipError_t launch_pack(const Geo &g, const void *input, void *xt, const void *weight, void *wp,
                       void *tab, bool transpose, hipStream_t s, const ClearList *clear) {
    if (g.B == 0) input = nullptr;  // weight packing only (also for an input read in place)
    switch (g.dtype) {
    case DCN2_F16: return pack_t<f16>(g, input, xt, weight, wp, tab, transpose, s, clear);
    case DCN2_BF16: return pack_t<bf16>(g, input, xt, weight, wp, tab, transpose, s, clear);
    default: return pack_t<float>(g, input, xt, weight, wp, tab, transpose, s, clear);
    }
}

}  // namespace dcn2
