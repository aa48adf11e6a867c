// Fused DCNv2 forward for gfx950: bilinear, mask-modulated sampling into LDS
// feeding a 32x32 MFMA GEMM, never materialising the column matrix.
//
// Reference: im2colcuda + dcn_bilinear_cuda write columns[B][C*kh*kw][N] to
// HBM (com.cu:119-195), then gemm_cuda reads them back (com.cu:46-117).  Here
// one workgroup owns a BM x BN output tile (all of Cout when Cout <= 256) and
// walks K in chunks of KC channels of one (tap, group):
//
//   for chunk ch:                       (double-buffered LDS stage sB[2])
//     load offset/mask of ch+3                       -- raw bits, used next step
//     issue A (weight) fragment loads for ch+1      -- global/L2, 16 B per lane
//     descriptors + corner gathers for ch+2          -- channels-last xt
//     MFMA over sB[ch&1]                             -- matrix cores
//     bilinear blend of ch+1 (gathered one step ago) -> sB[(ch+1)&1]
//     barrier
//
// so a corner gather has a whole step (an MFMA phase and a barrier) to land
// before its blend, and its offsets were loaded a step before that.
// Each sampled value is produced once per workgroup and reused by every output
// channel of the tile.
//
// Threads: 512 (8 waves) as WM x WN waves, each wave owning a 64x64 output
// sub-tile = 2x2 MFMA 32x32 blocks.  Sampling slot = (pixel, quarter of the
// chunk): 4 lanes cover one pixel's KC channels, so one corner of one pixel is
// read as a contiguous KC*sizeof(T)-byte run across 4 adjacent lanes.
#include <type_traits>

#include "dcn2_common.h"
#include "dcn2_sampler.h"
#include "dcn2_kernels.h"
#include "../../include/dcnv2_amd.h"

namespace dcn2 {

struct FwdParams {
    const void *xt, *wp, *tab, *offset, *mask, *bias;
    void *out;
    int H, W, Cout, kh, kw, sh, sw, ph, pw, dh, dw, G, Cgp, Ho, Wo, Kp;
    int ntiles, mtiles, tiles;  // pixel tiles per image, M tiles, B*ntiles*mtiles
    int out_vec;                // output rows can be written with 16-byte stores
};

template <typename T, int WM, int WN, int IB, int JB, bool MASK>
__global__ __launch_bounds__(512) void dcn2_fwd_kernel(const FwdParams p) {
    using M = Mma<T>;
    using frag = typename M::frag;
    constexpr int KC = M::KC, KPL = M::KPL, KSTEP = M::KSTEP, NKS = KC / KSTEP;
    constexpr int BN = 32 * JB * WN;            // each wave: 32*IB rows x 32*JB pixels
    constexpr int BM = 32 * IB * WM;
    static_assert(WM * WN == 8, "8 waves");
    constexpr int CPS = KC / 4;                 // channels per sampling slot
    constexpr int U4 = CPS * sizeof(T) / 16;    // 16-byte registers per corner per slot (2)
    constexpr int SPT = BN * 4 / 512;           // sampling slots per thread
    constexpr int LDK = KC + 16 / sizeof(T);    // LDS pitch (elements) of one pixel row
    static_assert(U4 == 2, "slot is 32 bytes per corner");

    // LDS: the two sampled-column stages during the K loop; afterwards the
    // same memory stages each wave's output tile for 16-byte row stores.
    constexpr int LDO = 32 * JB + 16 / sizeof(T);  // pitch (elements) of an output row
    constexpr size_t kStageBytes = sizeof(T) * 2 * BN * LDK;
    constexpr size_t kOutBytes = sizeof(T) == 2 ? sizeof(T) * 8 * 32 * IB * LDO : 0;
    __shared__ __attribute__((aligned(16))) char smem[kStageBytes > kOutBytes ? kStageBytes
                                                                              : kOutBytes];
    T(&sB)[2][BN][LDK] = *reinterpret_cast<T(*)[2][BN][LDK]>(smem);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave - wm * WN;
    // Tiles are numbered (image, pixel tile, M tile) and handed to XCDs in
    // contiguous ranges: consecutive workgroup ids go round-robin over the 8
    // XCDs, so XCD x receives the ids x, x+8, ... and is given the x-th range.
    // Neighbouring tiles of one image then share that XCD's L2 for their
    // corner gathers.
    const int t = xcd_remap(blockIdx.x, p.tiles);
    const int mt = t % p.mtiles, nt = (t / p.mtiles) % p.ntiles, b = t / (p.mtiles * p.ntiles);
    const int n0 = nt * BN, m0 = mt * BM;
    const int N = p.Ho * p.Wo, KK = p.kh * p.kw, cs = p.G * p.Cgp;
    const int nch = p.Kp / KC, last = nch - 1;

    const T *__restrict__ xt = (const T *)p.xt + (size_t)b * p.H * p.W * cs;
    const T *__restrict__ offs = (const T *)p.offset + (size_t)b * p.G * KK * 2 * N;
    const T *__restrict__ msk = MASK ? (const T *)p.mask + (size_t)b * p.G * KK * N : nullptr;
    const ChunkEnt *__restrict__ tab = (const ChunkEnt *)p.tab;

    SampleGeo sg;
    sg.H = p.H; sg.W = p.W; sg.kh = p.kh; sg.kw = p.kw; sg.sh = p.sh; sg.sw = p.sw;
    sg.ph = p.ph; sg.pw = p.pw; sg.dh = p.dh; sg.dw = p.dw; sg.G = p.G; sg.Cgp = p.Cgp;
    sg.Wo = p.Wo; sg.N = N; sg.cs = cs; sg.KK = KK;

    // Chunk c lives in set c % 2 of every pipeline buffer: offset/mask bits
    // om, corner gathers smp, A fragments a and the LDS stage sB.  The loop
    // is unrolled by two so that every set index is a compile-time constant,
    // and stages past the last chunk re-read the last chunk (clamped table
    // index) instead of branching, so one step is one basic block and the
    // scheduler can interleave its MFMA with the VALU work of the next chunk.
    Sampler<T, SPT, MASK> smp[2];
    smp[0].init(tid);
    smp[1].init(tid);
    SlotOM<T, SPT> om[2];
    frag a[2][IB][NKS];

    auto ent = [&](int ch) __attribute__((always_inline)) { return tab[min(ch, last)]; };

    // Bilinear blend of sampler set SET, stored to LDS stage SET as
    // [pixel][channel] rows (the MFMA B-operand order).
    auto store_stage = [&](auto set_c) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value;
#pragma unroll
        for (int s = 0; s < SPT; ++s) {
            const int pl = (tid + s * 512) >> 2;
            uint4 *dst = reinterpret_cast<uint4 *>(&sB[SET][pl][smp[SET].q * CPS]);
#pragma unroll
            for (int u = 0; u < U4; ++u) {
                float v[16 / sizeof(T)];
                smp[SET].blend(s, u, v);
                dst[u] = pack16<T>(v);
            }
        }
    };

    // A (weight) fragments of rows m0 + wm*64 + i*32 + lane%32, packed in
    // fragment order (pack_weight_kernel layout 0): the fragment (row block
    // rb, chunk ch, step ks) is 64 lanes x KPL contiguous elements.
    const T *wfrag[IB];
#pragma unroll
    for (int i = 0; i < IB; ++i)
        wfrag[i] = (const T *)p.wp + ((size_t)((m0 + wm * 32 * IB + i * 32) / 32) * nch * NKS * 64 +
                                      lane) * KPL;
    auto load_a = [&](auto set_c, int ch) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value;
        const int c = min(ch, last) * NKS * 64 * KPL;
#pragma unroll
        for (int i = 0; i < IB; ++i)
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks)
                a[SET][i][ks] = *reinterpret_cast<const frag *>(wfrag[i] + c + ks * 64 * KPL);
    };

    // The accumulators start at the bias of their output row, so the
    // epilogue only rounds and stores.
    f32x16 acc[IB][JB];
    const T *bias = (const T *)p.bias;
#pragma unroll
    for (int i = 0; i < IB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + wm * 32 * IB + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const float bv = (bias && m < p.Cout) ? to_f32(bias[m]) : 0.0f;
#pragma unroll
            for (int j = 0; j < JB; ++j) acc[i][j][r] = bv;
        }

    auto mfma_chunk = [&](auto set_c) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value;
        frag bf[NKS][JB];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
            for (int j = 0; j < JB; ++j)
                bf[ks][j] = *reinterpret_cast<const frag *>(
                    &sB[SET][(wn * JB + j) * 32 + (lane & 31)][ks * KSTEP + (lane >> 5) * KPL]);
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
            for (int i = 0; i < IB; ++i)
#pragma unroll
                for (int j = 0; j < JB; ++j)
                    acc[i][j] = M::mma(a[SET][i][ks], bf[ks][j], acc[i][j]);
    };

    // One pipeline step for chunk ch, set S = ch % 2, O = S ^ 1:
    //   offset/mask bits of ch+3 -> om[O]     A fragments of ch+1 -> a[O]
    //   corner gathers of ch+2 (om[S]) -> smp[S]
    //   MFMA of ch (a[S], sB[S])              blend of ch+1 (smp[O]) -> sB[O]
    // Chunk-table entries of ch+2 and ch+3 are held in scalar registers and
    // the entry of ch+4 is fetched one step ahead, so no step starts by
    // waiting for a scalar load.
    ChunkEnt e2 = ent(2), e3 = ent(3);
    auto step = [&](auto s_c, int ch) __attribute__((always_inline)) {
        constexpr int S = decltype(s_c)::value;
        constexpr int O = S ^ 1;
        // Loads whose results the next step consumes go first, so that the
        // in-order load counter lets the next step wait for them without
        // also waiting for this step's corner gathers.
        smp[0].load_om(n0, e3.x, sg, tid, offs, msk, om[O]);
        load_a(std::integral_constant<int, O>{}, ch + 1);
        const ChunkEnt e4 = ent(ch + 4);
        __builtin_amdgcn_sched_barrier(0);
        smp[S].issue(e2, sg, xt, om[S]);
        mfma_chunk(std::integral_constant<int, S>{});
        store_stage(std::integral_constant<int, O>{});
        // Interleave: each MFMA (32 cycles of the matrix core) is followed by
        // a slice of the blend / descriptor VALU work and one LDS read.
        __builtin_amdgcn_sched_group_barrier(0x100, JB * NKS, 0);  // all B-fragment reads
#pragma unroll
        for (int i = 0; i < IB * JB * NKS; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
        }
        __syncthreads();
        e2 = e3;
        e3 = e4;
    };

    // Prologue: offset/mask bits of chunks 0, 1, 2; gathers of chunks 0 and
    // 1; chunk 0 blended into stage 0.
    {
        const ChunkEnt e0 = ent(0), e1 = ent(1);
        smp[0].load_om(n0, e0.x, sg, tid, offs, msk, om[0]);
        smp[0].load_om(n0, e1.x, sg, tid, offs, msk, om[1]);
        load_a(std::integral_constant<int, 0>{}, 0);
        smp[0].issue(e0, sg, xt, om[0]);
        smp[0].load_om(n0, e2.x, sg, tid, offs, msk, om[0]);
        smp[1].issue(e1, sg, xt, om[1]);
        store_stage(std::integral_constant<int, 0>{});
        __syncthreads();
    }
    int ch = 0;
    for (; ch + 1 < nch; ch += 2) {
        step(std::integral_constant<int, 0>{}, ch);
        step(std::integral_constant<int, 1>{}, ch + 1);
    }
    if (ch < nch) step(std::integral_constant<int, 0>{}, ch);

    // Epilogue: round to T and store NCHW.  For 2-byte types with aligned,
    // 8-divisible rows each wave stages its 32*IB x 32*JB tile in LDS (the K
    // loop's stages are free after its last barrier) and writes whole 16-byte
    // row segments; otherwise every lane stores its own elements.
    T *out = (T *)p.out + (size_t)b * p.Cout * N;
    if constexpr (sizeof(T) == 2) {
        if (p.out_vec) {
            T *so = reinterpret_cast<T *>(smem) + (size_t)wave * 32 * IB * LDO;
#pragma unroll
            for (int i = 0; i < IB; ++i)
#pragma unroll
                for (int j = 0; j < JB; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        so[(i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * LDO + j * 32 +
                           (lane & 31)] = from_f32<T>(acc[i][j][r]);
            // each row is 32*JB elements = 4*JB segments of 8; a wave
            // instruction covers 64 segments
            constexpr int SEG = 4 * JB, ROWS = 32 * IB;
#pragma unroll
            for (int it = 0; it < ROWS * SEG / 64; ++it) {
                const int sidx = it * 64 + lane;
                const int row = sidx / SEG, seg = sidx - row * SEG;
                const int m = m0 + wm * ROWS + row, n = n0 + wn * 32 * JB + seg * 8;
                const uint4 v = *reinterpret_cast<const uint4 *>(so + row * LDO + seg * 8);
                if (m < p.Cout && n < N)  // N % 8 == 0: a segment is all in or all out
                    *reinterpret_cast<uint4 *>(out + (size_t)m * N + n) = v;
            }
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < IB; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + wm * 32 * IB + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m >= p.Cout) continue;
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                const int n = n0 + (wn * JB + j) * 32 + (lane & 31);
                if (n < N) out[(size_t)m * N + n] = from_f32<T>(acc[i][j][r]);
            }
        }
    }
}

template <typename T, int WM, int WN, int IB, int JB>
static hipError_t launch_fwd_t(const Geo &g, const FwdParams &p0, hipStream_t s) {
    FwdParams p = p0;
    p.ntiles = ceil_div(g.N, 32 * JB * WN);
    p.mtiles = g.Mp / (32 * IB * WM);
    p.tiles = g.B * p.ntiles * p.mtiles;
    p.out_vec = (g.N % 8 == 0) && (((uintptr_t)p.out & 15) == 0);
    if (p.mask)
        dcn2_fwd_kernel<T, WM, WN, IB, JB, true><<<p.tiles, 512, 0, s>>>(p);
    else
        dcn2_fwd_kernel<T, WM, WN, IB, JB, false><<<p.tiles, 512, 0, s>>>(p);
    return hipGetLastError();
}

// Block tile 256x128 (8 waves of 64x64) when Cout > 128, else 128x128 (8
// waves of 64x32); both sample 128 pixels, one slot per thread.
template <typename T>
static hipError_t launch_fwd_dt(const Geo &g, const FwdParams &p, hipStream_t s) {
    if (g.BM == 256) return launch_fwd_t<T, 8, 1, 1, 4>(g, p, s);
    return launch_fwd_t<T, 2, 4, 2, 1>(g, p, s);
}

hipError_t launch_forward(const Geo &g, const void *xt, const void *wp, const void *tab,
                          const void *offset, const void *mask, const void *bias, void *out,
                          hipStream_t s) {
    if (g.B == 0) return hipSuccess;
    FwdParams p;
    p.xt = xt;
    p.wp = wp;
    p.tab = tab;
    p.offset = offset;
    p.mask = mask;
    p.bias = bias;
    p.out = out;
    p.H = g.H;
    p.W = g.W;
    p.Cout = g.Cout;
    p.kh = g.kh;
    p.kw = g.kw;
    p.sh = g.sh;
    p.sw = g.sw;
    p.ph = g.ph;
    p.pw = g.pw;
    p.dh = g.dh;
    p.dw = g.dw;
    p.G = g.G;
    p.Cgp = g.Cgp;
    p.Ho = g.Ho;
    p.Wo = g.Wo;
    p.Kp = g.Kp;
    switch (g.dtype) {
    case DCN2_F16: return launch_fwd_dt<f16>(g, p, s);
    case DCN2_BF16: return launch_fwd_dt<bf16>(g, p, s);
    default: return launch_fwd_dt<float>(g, p, s);
    }
}

}  // namespace dcn2
