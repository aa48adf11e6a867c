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
    int Mp;                     // padded output rows of the packed weight
    int ntiles, mtiles, tiles;  // pixel tiles per image, M tiles, B*ntiles*mtiles
    // Chunks and M tiles walked by this launch.  A launch covers the M tiles
    // [mt_base, mt_base + mtiles) and, per tile, the nch_eff = KK*cpw chunks
    // ch = tap*cpt + cb + i (i < cpw) of the packed K order (tap, group,
    // channel chunk), cpt chunks per tap.  One launch per weight group walks
    // only that group's rows and chunks; an ungrouped launch has cb = 0 and
    // cpw = cpt, i.e. every chunk.
    int mt_base, cpt, cpw, cb, nch_eff;
    int out_vec;                // output rows can be written with 16-byte stores
    int out_nhwc;               // output is channels-last [B][Ho][Wo][Cout]
    long long off_bs, msk_bs;   // offset / mask elements between images
    int msk_logit;              // mask buffer holds logits (see mask_value)
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
    const int n0 = nt * BN, m0 = (p.mt_base + mt) * BM;
    const int N = p.Ho * p.Wo, KK = p.kh * p.kw, cs = p.G * p.Cgp;
    const int nch_all = p.Kp / KC;         // chunks of the packed weight rows
    const int nch = p.nch_eff, last = nch - 1;  // chunks walked (see FwdParams)
    // j-th chunk of the walk -> packed chunk index
    auto chmap = [&](int j) __attribute__((always_inline)) {
        j = min(j, last);
        const int tap = j / p.cpw;
        return tap * p.cpt + p.cb + (j - tap * p.cpw);
    };

    const T *__restrict__ xt = (const T *)p.xt + (size_t)b * p.H * p.W * cs;
    const T *__restrict__ offs = (const T *)p.offset + (size_t)b * p.off_bs;
    const T *__restrict__ msk = MASK ? (const T *)p.mask + (size_t)b * p.msk_bs : nullptr;
    const ChunkEnt *__restrict__ tab = (const ChunkEnt *)p.tab;

    SampleGeo sg;
    sg.H = p.H; sg.W = p.W; sg.kh = p.kh; sg.kw = p.kw; sg.sh = p.sh; sg.sw = p.sw;
    sg.ph = p.ph; sg.pw = p.pw; sg.dh = p.dh; sg.dw = p.dw; sg.G = p.G; sg.Cgp = p.Cgp;
    sg.Wo = p.Wo; sg.N = N; sg.cs = cs; sg.KK = KK; sg.msk_logit = p.msk_logit;

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

    auto ent = [&](int ch) __attribute__((always_inline)) { return tab[chmap(ch)]; };

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
        wfrag[i] = (const T *)p.wp + ((size_t)((m0 + wm * 32 * IB + i * 32) / 32) * nch_all * NKS * 64 +
                                      lane) * KPL;
    auto load_a = [&](auto set_c, int ch) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value;
        const int c = chmap(ch) * NKS * 64 * KPL;
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

    // Epilogue: round to T and store.  For 2-byte types with an NCHW output
    // of aligned, 8-divisible rows each wave stages its 32*IB x 32*JB tile in
    // LDS (the K loop's stages are free after its last barrier) and writes
    // whole 16-byte row segments; otherwise every lane stores its own elements.
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
    // element stores: NCHW (m * N + n) or channels-last (n * Cout + m)
    const size_t ms = p.out_nhwc ? 1 : (size_t)N, ns = p.out_nhwc ? (size_t)p.Cout : 1;
#pragma unroll
    for (int i = 0; i < IB; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + wm * 32 * IB + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m >= p.Cout) continue;
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                const int n = n0 + (wn * JB + j) * 32 + (lane & 31);
                if (n < N) out[m * ms + n * ns] = from_f32<T>(acc[i][j][r]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Warp-specialised forward for 2-byte types (f16, bf16).
//
// The 8 waves of a workgroup split into two roles that run concurrently on
// every SIMD (waves w and w+4 share SIMD w % 4):
//   waves 0-3  MFMA waves: each owns 32*IB output rows x all BN = 128 pixels
//              of the tile, loads its weight fragments from the fragment-
//              ordered packed weight and runs the 32x32x16 MFMAs over the LDS
//              stage of the current chunk;
//   waves 4-7  sampler waves: the bilinear descriptor of every (pixel, chunk)
//              is computed by one pair of sampler threads three chunks ahead
//              and put in an LDS ring; two chunks ahead every sampler lane
//              reads the descriptors of its four pixels and issues their
//              corner gathers; one chunk ahead it blends them into the free
//              LDS stage.
// One barrier per chunk hands a stage from the samplers to the MFMA waves.
// The matrix cores and the blend VALU then overlap across waves instead of
// alternating inside one wave.  The workgroup is persistent: it walks its
// tiles back to back (tile k+1's sampling pipeline starts while tile k's last
// chunk is multiplied), with tiles dispatched XCD-aware as in xcd_remap.
//
// Gather lane map: 8 consecutive lanes read the 8 16-byte pieces of one
// corner of one pixel (64 channels x 2 bytes = one 128-byte line), so a wave
// instruction touches 8 lines.  Measured on MI355X, L2-resident 128-byte
// lines stream at ~50 B/clk/CU this way against ~30 B/clk/CU with 2 lanes
// per line: the vector L1 handles about one line per clock per instruction.
// ---------------------------------------------------------------------------

// Descriptor of one (pixel, chunk) in the LDS ring: the four corner offsets
// (bytes, 0 outside the image) and the four mask-folded corner weights as
// fp32 bits.  Half h (16 bytes) holds corners 2h and 2h+1.
struct RingHalf {
    int o0, o1;
    uint32_t w0, w1;
};
struct RingDesc {
    RingHalf h[2];
};

// Bilinear blend of one 16-byte piece (8 channels) of the four corners:
// fp32 weights, fp32 products and sums, one rounding to T at the end, as the
// reference's sampler computes in fp32 and rounds its columns once
// (com.cu:119-148, 83, 87).  For f16 the conversions fold into mixed-precision
// FMAs (f16 source, fp32 accumulator).
template <typename T> struct Blend8 {
    static __device__ __forceinline__ uint4 weights(const float (&w)[4]) {
        return make_uint4(__float_as_uint(w[0]), __float_as_uint(w[1]), __float_as_uint(w[2]),
                          __float_as_uint(w[3]));
    }
    static __device__ __forceinline__ uint4 run(const uint4 (&r)[4], uint4 wd) {
        const float w[4] = {__uint_as_float(wd.x), __uint_as_float(wd.y), __uint_as_float(wd.z),
                            __uint_as_float(wd.w)};
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float v[8];
            Unpack<T>::run(r[q], v);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(w[q], v[e], acc[e]);
        }
        return pack16<T>(acc);
    }
};

// Rows of the LDS bias table of the warp-specialised forward.
constexpr int kBiasRows = 1024;

// MASK: 0 no mask (all ones), 1 mask values, 2 mask logits (sigmoid on load);
// a compile-time mode keeps the descriptor code free of branches, so it can
// be scheduled between the MFMAs.  ONHWC: channels-last output.
template <typename T, int IB, int MASK, bool ONHWC>
__global__ __launch_bounds__(512) void dcn2_fwd_ws_kernel(const FwdParams p) {
    using M = Mma<T>;
    using frag = typename M::frag;
    constexpr int KC = 64, KPL = 8, KSTEP = 16, NKS = 4;
    constexpr int BN = 128, JB = 4;      // tile pixels; 32-pixel blocks per MFMA wave
    constexpr int ROWS = 32 * IB;        // output rows per MFMA wave
    constexpr int LDK = KC + 8;          // stage pitch (elements): 144 B, conflict-free fragments
    constexpr int LDO = BN + 8;          // epilogue staging pitch (elements), NCHW: [row][pixel]
    constexpr int LDC = ROWS + 8;        // the same, channels-last: [pixel][row]
    static_assert(sizeof(T) == 2, "2-byte types only");
    constexpr int kOutElems = ONHWC ? BN * LDC : ROWS * LDO;  // per MFMA wave

    __shared__ __attribute__((aligned(16))) T sB[2][BN][LDK];
    __shared__ __attribute__((aligned(16))) T sO[4][kOutElems];
    __shared__ RingDesc ring[2][BN];
    __shared__ __attribute__((aligned(16))) float sBias[kBiasRows];

    const int tid = threadIdx.x, lane = tid & 63;
    // Role election: the MFMA waves must sit on four different SIMDs (two
    // MFMA waves on one SIMD would halve the matrix rate), and the hardware
    // does not promise which SIMD a wave of the workgroup lands on.  At this
    // register count a SIMD holds at most two of the eight waves, so every
    // SIMD holds exactly two: the first to arrive takes the MFMA role and
    // the other the sampler role; rw (0..3) = SIMD id indexes the role.
    __shared__ int simd_seen[4];
    if (tid < 4) simd_seen[tid] = 0;
    __syncthreads();
    int rw;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID, 4, 2)" : "=s"(rw));
    int rank = 0;
    if (lane == 0) rank = atomicAdd(&simd_seen[rw], 1);
    const bool mfma_role = __builtin_amdgcn_readfirstlane(__shfl(rank, 0)) == 0;
    const int N = p.Ho * p.Wo, KK = p.kh * p.kw, cs = p.G * p.Cgp;
    const int nch_all = p.Kp / KC;              // chunks of the packed weight rows
    const int nch = p.nch_eff, last = nch - 1;  // chunks walked per tile (see FwdParams)
    const int ntile = p.tiles, G = gridDim.x;
    // this workgroup's tiles are the dispatch ids blockIdx.x + k*G, k = 0..
    const int my_tiles = blockIdx.x < ntile ? (ntile - 1 - blockIdx.x) / G + 1 : 0;
    const int S = my_tiles * nch;  // pipeline steps (chunks) of this workgroup
    // The chunk table is read through the constant address space: with a
    // wave-uniform index that makes every read a scalar load, which the
    // vector-memory counter (and so the corner gathers in flight) never waits on.
    typedef const __attribute__((address_space(4))) int *ConstTab;
    const ConstTab tabi = (ConstTab)(uintptr_t)p.tab;
    auto tab_ent = [&](int ch) __attribute__((always_inline)) {
        return make_int4(tabi[4 * ch], tabi[4 * ch + 1], tabi[4 * ch + 2], tabi[4 * ch + 3]);
    };

    // Pipeline cursor: position (k-th tile of this workgroup, chunk ch) of
    // one pipeline point, advanced by one chunk per step.  Positions past the
    // last tile stay on the last tile, so look-ahead loads remain in bounds.
    // Every workgroup walks the chunks of its tiles in the same cyclic order
    // but from its own starting chunk rot, so the tile ends (and the output
    // stores they issue) of different workgroups are spread over time instead
    // of hitting HBM all at once.  j counts the chunks done in the tile.
    const int rot = blockIdx.x % nch;
    // (tap, i): position in the chunk walk, ch = tap*cpt + cb + i the packed chunk
    struct Cursor { int k, j, tap, i, ch, b, n0, m0; };
    // Cursor fields are wave-uniform; readfirstlane keeps them in SGPRs.
    // Otherwise (the role branch is divergent code to the compiler) they
    // live in VGPRs, the chunk-table reads become vector loads, and waiting
    // for one of those waits for every corner gather issued before it.
    auto uni = [](int v) __attribute__((always_inline)) { return __builtin_amdgcn_readfirstlane(v); };
    auto set_tile = [&](Cursor &c) __attribute__((always_inline)) {
        const int t = xcd_remap(blockIdx.x + min(c.k, my_tiles - 1) * G, ntile);
        const int mt = t % p.mtiles, r = t / p.mtiles;
        c.n0 = uni((r % p.ntiles) * BN);
        c.b = uni(r / p.ntiles);
        c.m0 = uni((p.mt_base + mt) * 4 * ROWS);
    };
    auto cursor = [&](int g) __attribute__((always_inline)) {
        Cursor c;
        c.k = uni(g / nch);
        c.j = uni(g - c.k * nch);
        const int r = c.j + rot < nch ? c.j + rot : c.j + rot - nch;
        c.tap = uni(r / p.cpw);
        c.i = uni(r - c.tap * p.cpw);
        c.ch = uni(c.tap * p.cpt + p.cb + c.i);
        set_tile(c);
        return c;
    };
    // Advances c by one chunk; on a tile change refreshes the tile fields and
    // runs on_tile() to refresh the caller's per-tile state.  The empty
    // volatile asm keeps the (rare) tile change a real branch: if-converted,
    // its divisions would run every step on the scalar unit.
    auto advance = [&](Cursor &c, auto &&on_tile) __attribute__((always_inline)) {
        // next chunk of the walk: i + 1, else the next tap (the walk wraps at KK)
        const bool wrap_i = c.i + 1 == p.cpw, wrap_t = wrap_i && c.tap + 1 == KK;
        c.ch = uni(wrap_t ? p.cb : (wrap_i ? c.ch + 1 + p.cpt - p.cpw : c.ch + 1));
        c.tap = uni(wrap_t ? 0 : (wrap_i ? c.tap + 1 : c.tap));
        c.i = uni(wrap_i ? 0 : c.i + 1);
        c.j = uni(c.j + 1);
        if (c.j == nch) {
            asm volatile("");
            c.j = 0;
            c.k = uni(c.k + 1);
            set_tile(c);
            on_tile();
        }
    };
    auto no_tile = [] {};

    // Byte offset the descriptors give a corner outside the image: past the
    // image's channels-last input, so the sampler's buffer load returns 0
    // without a memory access (the host keeps it and every in-image offset
    // plus the chunk's channel offset below 2^32).
    const uint32_t img_bytes = (uint32_t)((size_t)p.H * p.W * cs * sizeof(T));

    if (mfma_role) {
        // ------------------------------------------------------------ MFMA waves
        // Two sets of A fragments: the set of chunk g+1 is loaded at the top
        // of step g, ahead of the MFMAs of chunk g, so it has a whole step to
        // land.  (Left to itself the scheduler sinks the loads to the end of
        // the step, which exposes their full latency every step.)
        frag a[2][IB][NKS];

        // The MFMA waves also compute the bilinear descriptors, three chunks
        // ahead, into the LDS ring: their instruction stream waits on the
        // matrix core most of the step, while a sampler wave can issue only
        // one instruction per cycle slot and is the longer of the two roles.
        // Threads 2p, 2p+1 (st = rw*64 + lane) both evaluate pixel p of the
        // descriptor chunk and write half of it each (no divergent branch in
        // the step, so the compiler's load counting stays exact).
        const int st = rw * 64 + lane;  // 0..255
        const int dpix = st >> 1, dhalf = st & 1;
        // Offset/mask bits of one chunk for pixel dpix (kept raw until used)
        // with the pixel's output position in the tile they belong to: loaded
        // in step g for chunk g+4, after the descriptors of chunk g+3 have
        // used the previous load, so each load has a whole step to land.
        struct OmBits {
            int n, by, bx;
            T dy, dx, m;
        };
        OmBits om;
        // Per-tile state of the offset-load point: offset/mask planes of the
        // image and the output position of pixel dpix.
        const T *offb, *mskb;
        int n_t, nn_t, by_t, bx_t;
        auto set_om_tile = [&](const Cursor &c) __attribute__((always_inline)) {
            offb = (const T *)p.offset + (size_t)c.b * p.off_bs;
            mskb = MASK ? (const T *)p.mask + (size_t)c.b * p.msk_bs : nullptr;
            n_t = c.n0 + dpix;
            nn_t = n_t < N ? n_t : 0;
            const int oy = nn_t / p.Wo, ox = nn_t - oy * p.Wo;
            by_t = oy * p.sh - p.ph;
            bx_t = ox * p.sw - p.pw;
        };
        auto load_om = [&](const Cursor &c) __attribute__((always_inline)) {
            const int plane = tabi[4 * c.ch];
            om.n = n_t;
            om.by = by_t;
            om.bx = bx_t;
            const size_t ob = (size_t)plane * 2 * N + nn_t;
            om.dy = offb[ob];
            om.dx = offb[ob + N];
            if constexpr (MASK) om.m = mskb[(size_t)plane * N + nn_t];
        };
        // descriptor of pixel dpix at cursor c from om -> ring slot R (this
        // thread's half); corner offsets in bytes, img_bytes outside
        auto put_desc = [&](int R, const Cursor &c) __attribute__((always_inline)) {
            const ChunkEnt e = tab_ent(c.ch);
            const float y = (float)(om.by + e.y) + to_f32(om.dy);
            const float x = (float)(om.bx + e.z) + to_f32(om.dx);
            float mv = 1.0f;
            if constexpr (MASK == 1) mv = to_f32(om.m);
            if constexpr (MASK == 2) mv = 1.0f / (1.0f + __expf(-to_f32(om.m)));
            mv = om.n < N ? mv : 0.0f;  // pixels past N sample 0
            const SamplePos sp = sample_pos(y, x, p.H, p.W);
            const Corners cr = make_corners(sp, mv, p.W, cs);
            const uint4 wq = Blend8<T>::weights(cr.w);
            const bool vy = dhalf ? sp.vy1 : sp.vy0;
            RingHalf hd;
            // (bit selects: written as conditional expressions these became a
            // divergent branch, which split the step's scheduling region and
            // left the descriptor VALU after the MFMAs instead of between them)
            const int oa = (dhalf ? cr.off[2] : cr.off[0]) * (int)sizeof(T);
            const int ob = (dhalf ? cr.off[3] : cr.off[1]) * (int)sizeof(T);
            const int ma = -(int)(vy && sp.vx0), mb = -(int)(vy && sp.vx1);
            hd.o0 = (oa & ma) | ((int)img_bytes & ~ma);
            hd.o1 = (ob & mb) | ((int)img_bytes & ~mb);
            hd.w0 = dhalf ? wq.z : wq.x;
            hd.w1 = dhalf ? wq.w : wq.y;
            ring[R][dpix].h[dhalf] = hd;
        };
        f32x16 acc[IB][JB];
        const T *bias = (const T *)p.bias;
        const T *wbase = (const T *)p.wp + (size_t)lane * KPL;
        // Bias of this wave's rows of every M tile in LDS (fp32, 0 past Cout;
        // the host guarantees Mp <= kBiasRows), so starting a tile never waits
        // on a global load queued behind the A loads in flight.  Each wave
        // writes and reads only its own rows: no barrier needed.
        for (int m = lane; m < p.Mp; m += 64)
            if ((m / ROWS) % 4 == rw) sBias[m] = (bias && m < p.Cout) ? to_f32(bias[m]) : 0.0f;
        // The MFMAs compute the transposed tile D^T[n][m] (the weight
        // fragment is the B operand, the sampled columns the A operand; both
        // operands have the same register layout), so lane l holds output
        // row m = i*32 + l%32 and, in acc[r], pixel n = j*32 + 8*(r/4) +
        // 4*(l/32) + r%4: four consecutive pixels of one row per r/4.
        // (filled as 64-bit register pairs: half the move instructions).
        // With a channels-last output the MFMAs compute D[m][n] instead
        // (weight fragment as the A operand): lane l then holds pixel
        // n = j*32 + l%32 and, in acc[r], output row m = i*32 + 8*(r/4) +
        // 4*(l/32) + r%4, four consecutive channels of one pixel per r/4.
        auto init_acc = [&](int m0) __attribute__((always_inline)) {
            if constexpr (ONHWC) {
#pragma unroll
                for (int i = 0; i < IB; ++i)
#pragma unroll
                    for (int rq = 0; rq < 4; ++rq) {
                        const f32x4 b4 = *reinterpret_cast<const f32x4 *>(
                            &sBias[m0 + rw * ROWS + i * 32 + 8 * rq + 4 * (lane >> 5)]);
#pragma unroll
                        for (int j = 0; j < JB; ++j)
#pragma unroll
                            for (int e = 0; e < 4; ++e) acc[i][j][4 * rq + e] = b4[e];
                    }
            } else {
                typedef unsigned long long u64x8 __attribute__((ext_vector_type(8)));
#pragma unroll
                for (int i = 0; i < IB; ++i) {
                    const uint32_t bb = __float_as_uint(sBias[m0 + rw * ROWS + i * 32 + (lane & 31)]);
                    const unsigned long long b2 = ((unsigned long long)bb << 32) | bb;
#pragma unroll
                    for (int j = 0; j < JB; ++j) acc[i][j] = __builtin_bit_cast(f32x16, u64x8(b2));
                }
            }
        };
        // A fragments at cursor c: rows m0 + rw*ROWS + i*32 + lane%32 of chunk
        // c.ch; wrow = first fragment of this wave's rows of the next tile's M block
        const T *wrow;
        auto set_wrow = [&](const Cursor &c) __attribute__((always_inline)) {
            wrow = wbase + (size_t)((c.m0 + rw * ROWS) / 32) * nch_all * NKS * 64 * KPL;
        };
        auto load_a = [&](auto set_c, const Cursor &c) __attribute__((always_inline)) {
            constexpr int SET = decltype(set_c)::value;
            const T *w0 = wrow + (size_t)c.ch * NKS * 64 * KPL;
#pragma unroll
            for (int i = 0; i < IB; ++i)
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks)
                    a[SET][i][ks] = *reinterpret_cast<const frag *>(
                        w0 + ((size_t)i * nch_all * NKS + ks) * 64 * KPL);
        };
        auto mfma_stage = [&](auto set_c) __attribute__((always_inline)) {
            constexpr int SET = decltype(set_c)::value;
            frag bf[2][JB];
#pragma unroll
            for (int j = 0; j < JB; ++j)
                bf[0][j] = *reinterpret_cast<const frag *>(
                    &sB[SET][j * 32 + (lane & 31)][(lane >> 5) * KPL]);
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                if (ks + 1 < NKS) {
#pragma unroll
                    for (int j = 0; j < JB; ++j)
                        bf[(ks + 1) & 1][j] = *reinterpret_cast<const frag *>(
                            &sB[SET][j * 32 + (lane & 31)][(ks + 1) * KSTEP + (lane >> 5) * KPL]);
                }
#pragma unroll
                for (int i = 0; i < IB; ++i)
#pragma unroll
                    for (int j = 0; j < JB; ++j) {
                        if constexpr (ONHWC)
                            acc[i][j] = M::mma(a[SET][i][ks], bf[ks & 1][j], acc[i][j]);
                        else
                            acc[i][j] = M::mma(bf[ks & 1][j], a[SET][i][ks], acc[i][j]);
                    }
            }
        };
        // Output tile of this wave: round to T, stage in LDS, then 16-byte
        // stores (or, for an output whose rows 16-byte stores cannot cover, a
        // plain loop of element stores from the staged tile).  Stores go
        // through a buffer over the image's output: a 16-byte piece outside
        // the output gets an offset past the buffer and is dropped, so no
        // store sits in a branch.
        typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
        auto store_tile = [&](const Cursor &c) __attribute__((always_inline)) {
            T *out = (T *)p.out + (size_t)c.b * p.Cout * N;
            const uint32_t obytes = (uint32_t)((size_t)p.Cout * N * sizeof(T));
            const __amdgpu_buffer_rsrc_t ors =
                __builtin_amdgcn_make_buffer_rsrc(out, (short)0, (int)obytes, 0x00020000);
            const int mw = c.m0 + rw * ROWS;  // first output row of this wave
            if constexpr (ONHWC) {
                // [pixel][row] staging: four consecutive rows of a pixel -> one
                // 8-byte LDS write; then each pixel's ROWS channels are
                // ROWS/8 16-byte pieces, 8 lanes per pixel per instruction
                T(&so)[BN][LDC] = *reinterpret_cast<T(*)[BN][LDC]>(sO[rw]);
#pragma unroll
                for (int i = 0; i < IB; ++i)
#pragma unroll
                    for (int j = 0; j < JB; ++j)
#pragma unroll
                        for (int rq = 0; rq < 4; ++rq) {
                            T v4[4];
#pragma unroll
                            for (int e = 0; e < 4; ++e) v4[e] = from_f32<T>(acc[i][j][rq * 4 + e]);
                            *reinterpret_cast<uint2 *>(&so[j * 32 + (lane & 31)][i * 32 + 8 * rq + 4 * (lane >> 5)]) =
                                __builtin_bit_cast(uint2, v4);
                        }
                if (p.out_vec) {
                    constexpr int SEG = ROWS / 8, PPI = 64 / SEG;
                    const int seg = lane % SEG, q = lane / SEG;
                    const int m = mw + seg * 8;
#pragma unroll
                    for (int it = 0; it < BN / PPI; ++it) {
                        const int pl = it * PPI + q, n = c.n0 + pl;
                        const uint4 v = *reinterpret_cast<const uint4 *>(&so[pl][seg * 8]);
                        const uint32_t off =
                            m < p.Cout && n < N
                                ? (uint32_t)(((unsigned)n * (unsigned)p.Cout + (unsigned)m) * sizeof(T))
                                : obytes;
                        __builtin_amdgcn_raw_buffer_store_b128(u32x4{v.x, v.y, v.z, v.w}, ors, (int)off, 0, 0);
                    }
                } else {
#pragma unroll 1
                    for (int idx = lane; idx < ROWS * BN; idx += 64) {
                        const int pl = idx / ROWS, row = idx % ROWS;
                        const int m = mw + row, n = c.n0 + pl;
                        if (m < p.Cout && n < N) out[(size_t)n * p.Cout + m] = so[pl][row];
                    }
                }
            } else {
                // [row][pixel] staging: four consecutive pixels of a row -> one
                // 8-byte LDS write
                T(&so)[ROWS][LDO] = *reinterpret_cast<T(*)[ROWS][LDO]>(sO[rw]);
#pragma unroll
                for (int i = 0; i < IB; ++i)
#pragma unroll
                    for (int j = 0; j < JB; ++j)
#pragma unroll
                        for (int rq = 0; rq < 4; ++rq) {
                            T v4[4];
#pragma unroll
                            for (int e = 0; e < 4; ++e) v4[e] = from_f32<T>(acc[i][j][rq * 4 + e]);
                            *reinterpret_cast<uint2 *>(&so[i * 32 + (lane & 31)][j * 32 + 8 * rq + 4 * (lane >> 5)]) =
                                __builtin_bit_cast(uint2, v4);
                        }
                if (p.out_vec) {
                    // a wave instruction covers 64 / SEG whole rows of SEG
                    // 16-byte segments (N % 8 == 0: a segment is all in or out)
                    constexpr int SEG = BN / 8, RPI = 64 / SEG;
                    const int seg = lane % SEG, r0 = lane / SEG;
                    const int n = c.n0 + seg * 8;
#pragma unroll
                    for (int it = 0; it < ROWS / RPI; ++it) {
                        const int m = mw + it * RPI + r0;
                        const uint4 v = *reinterpret_cast<const uint4 *>(&so[it * RPI + r0][seg * 8]);
                        const uint32_t off =
                            m < p.Cout && n < N
                                ? (uint32_t)(((unsigned)m * (unsigned)N + (unsigned)n) * sizeof(T))
                                : obytes;
                        __builtin_amdgcn_raw_buffer_store_b128(u32x4{v.x, v.y, v.z, v.w}, ors, (int)off, 0, 0);
                    }
                } else {
#pragma unroll 1
                    for (int idx = lane; idx < ROWS * BN; idx += 64) {
                        const int row = idx / BN, col = idx % BN;
                        const int m = mw + row, n = c.n0 + col;
                        if (m < p.Cout && n < N) out[(size_t)m * N + n] = so[row][col];
                    }
                }
            }
        };
        // chunk being multiplied, chunk loaded next, descriptor chunk, offset chunk
        Cursor cur = cursor(0), nxt = cursor(1), cd = cursor(3), co = cursor(4);
        // Step g (S_ = g % 2): A fragments of g+1 first, then the MFMAs of g
        // with the descriptors of g+3 (ring slot (g+3) % 2, from the offsets
        // loaded one step earlier) in between, then the offsets of g+4.
        auto step = [&](auto s_c) __attribute__((always_inline)) {
            constexpr int S_ = decltype(s_c)::value;
            load_a(std::integral_constant<int, S_ ^ 1>{}, nxt);
            __builtin_amdgcn_sched_barrier(0);
            mfma_stage(std::integral_constant<int, S_>{});
            put_desc(S_ ^ 1, cd);
            load_om(co);
            // Interleave (one scheduling region: the step has no divergent
            // branch up to here): the B fragments of ks 0 and 1, then per ks
            // eight MFMAs with up to three VALU instructions of the
            // descriptors after each, and the B fragments of ks + 2.  The MFMA
            // pipe holds the wave's issue for most of the step, so the
            // descriptor arithmetic rides in its gaps.
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
                for (int m = 0; m < IB * JB; ++m) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                }
                if (ks + 2 < NKS) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
            }
            if (cur.j == last) {  // tile done: write it, start the next one at its bias
                store_tile(cur);
                if (nxt.k < my_tiles) init_acc(nxt.m0);
            }
            advance(cur, no_tile);
            advance(nxt, [&] { set_wrow(nxt); });
            advance(cd, no_tile);
            advance(co, [&] { set_om_tile(co); });
            __syncthreads();
        };
        init_acc(cur.m0);
        set_wrow(cur);
        load_a(std::integral_constant<int, 0>{}, cur);
        set_wrow(nxt);
        // prologue: descriptors of chunks 0 and 1 (ring slots 0, 1) before
        // the first barrier; chunk 2 into slot 0 once the samplers have read
        // it (second barrier); offsets of chunk 3 for step 0
        {
            const Cursor c0 = cursor(0), c1 = cursor(1), c2 = cursor(2), c3 = cursor(3);
            set_om_tile(c0);
            load_om(c0);
            put_desc(0, c0);
            set_om_tile(c1);
            load_om(c1);
            put_desc(1, c1);
            set_om_tile(c2);
            load_om(c2);
            __syncthreads();
            __syncthreads();
            put_desc(0, c2);
            set_om_tile(c3);
            load_om(c3);
            __syncthreads();
            set_om_tile(co);
        }
        int g = 0;
        for (; g + 1 < S; g += 2) {
            step(std::integral_constant<int, 0>{});
            step(std::integral_constant<int, 1>{});
        }
        if (g < S) step(std::integral_constant<int, 0>{});
    } else {
        // --------------------------------------------------------- sampler waves
        const int cg = lane & 7;                      // 16-byte piece (8 channels) of a corner
        const int pbase = rw * 32 + (lane >> 3);      // slot s covers pixel pbase + 8*s
        uint4 raw[2][4][4];   // [set][slot][corner]
        uint4 wts[2][4];      // [set][slot] corner weights

        // Per-tile state of the gather point: a buffer resource over the
        // image's channels-last input (byte offsets are 32-bit, and a read
        // past the image returns 0).
        __amdgpu_buffer_rsrc_t xrs;
        auto set_x_tile = [&](const Cursor &c) __attribute__((always_inline)) {
            const T *xb = (const T *)p.xt + (size_t)c.b * p.H * p.W * cs;
            xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<T *>(xb), (short)0, (int)img_bytes,
                                                    0x00020000);
        };
        // corner gathers of the four slots at cursor c (descriptors in ring slot R) -> set SET
        typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
        auto gather = [&](int off, int soff) __attribute__((always_inline)) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
                xrs, (int)((unsigned)off + (unsigned)cg * 16u), soff, 0);
            return make_uint4(v.x, v.y, v.z, v.w);
        };
        auto issue = [&](auto set_c, int R, const Cursor &c) __attribute__((always_inline)) {
            constexpr int SET = decltype(set_c)::value;
            const int soff = tabi[4 * c.ch + 3] * (int)sizeof(T);  // chunk's first channel
#pragma unroll
            for (int sl = 0; sl < 4; ++sl) {
                const RingDesc d = ring[R][pbase + 8 * sl];
                wts[SET][sl] = make_uint4(d.h[0].w0, d.h[0].w1, d.h[1].w0, d.h[1].w1);
                raw[SET][sl][0] = gather(d.h[0].o0, soff);
                raw[SET][sl][1] = gather(d.h[0].o1, soff);
                raw[SET][sl][2] = gather(d.h[1].o0, soff);
                raw[SET][sl][3] = gather(d.h[1].o1, soff);
            }
        };
        auto blend_store = [&](auto set_c) __attribute__((always_inline)) {
            constexpr int SET = decltype(set_c)::value;
#pragma unroll
            for (int sl = 0; sl < 4; ++sl)
                *reinterpret_cast<uint4 *>(&sB[SET][pbase + 8 * sl][cg * 8]) =
                    Blend8<T>::run(raw[SET][sl], wts[SET][sl]);
        };
        // Chunk c uses ring slot, gather set and LDS stage c & 1.  Step g:
        //   gathers of g+2 (ring (g+2)&1) -> set g&1;
        //   blend of g+1 (set (g+1)&1) -> stage (g+1)&1;
        // with the gathers interleaved into the blend so that the vector
        // memory pipe is fed through the whole step.
        Cursor ci = cursor(2);  // issue point
        auto step = [&](auto s_c) __attribute__((always_inline)) {
            constexpr int S_ = decltype(s_c)::value;
            issue(std::integral_constant<int, S_>{}, S_, ci);
            blend_store(std::integral_constant<int, S_ ^ 1>{});
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // ring reads
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x020, 4, 0);  // gathers
                __builtin_amdgcn_sched_group_barrier(0x002, 30, 0);  // VALU
            }
            advance(ci, [&] { set_x_tile(ci); });
            __syncthreads();
        };
        // (S >= 1: the grid never exceeds the tile count)
        // after the first barrier the ring holds the descriptors of chunks 0
        // and 1
        {
            const Cursor c0 = cursor(0), c1 = cursor(1);
            __syncthreads();
            set_x_tile(c0);
            issue(std::integral_constant<int, 0>{}, 0, c0);
            __syncthreads();  // ring slot 0 is read: chunk 2 may replace chunk 0
            set_x_tile(c1);
            issue(std::integral_constant<int, 1>{}, 1, c1);
            blend_store(std::integral_constant<int, 0>{});
            __syncthreads();
            set_x_tile(ci);
        }
        int g = 0;
        for (; g + 1 < S; g += 2) {
            step(std::integral_constant<int, 0>{});
            step(std::integral_constant<int, 1>{});
        }
        if (g < S) step(std::integral_constant<int, 0>{});
    }
}

template <typename T, int WM, int WN, int IB, int JB>
static hipError_t launch_fwd_t(const Geo &g, const FwdParams &p0, hipStream_t s) {
    FwdParams p = p0;
    p.ntiles = ceil_div(g.N, 32 * JB * WN);
    p.tiles = g.B * p.ntiles * p.mtiles;
    p.out_vec = !p.out_nhwc && (g.N % 8 == 0) && (((uintptr_t)p.out & 15) == 0);
    if (p.mask)
        dcn2_fwd_kernel<T, WM, WN, IB, JB, true><<<p.tiles, 512, 0, s>>>(p);
    else
        dcn2_fwd_kernel<T, WM, WN, IB, JB, false><<<p.tiles, 512, 0, s>>>(p);
    return hipGetLastError();
}

// Warp-specialised kernel for 2-byte types: persistent grid of one
// workgroup per CU (at most one tile per workgroup more than the average).
template <typename T, int IB>
static hipError_t launch_fwd_ws(const Geo &g, const FwdParams &p0, hipStream_t s) {
    FwdParams p = p0;
    p.ntiles = ceil_div(g.N, 128);
    p.tiles = g.B * p.ntiles * p.mtiles;
    // 16-byte pieces of NCHW rows need N % 8 == 0, of channels-last pixels Cout % 8 == 0
    p.out_vec = (p.out_nhwc ? g.Cout % 8 == 0 : g.N % 8 == 0) && (((uintptr_t)p.out & 15) == 0);
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        ncu <= 0)
        ncu = 256;
    const int grid = p.tiles < ncu ? p.tiles : ncu;
    const int mode = p.mask ? (p.msk_logit ? 2 : 1) : 0;
    if (p.out_nhwc) {
        if (mode == 2) dcn2_fwd_ws_kernel<T, IB, 2, true><<<grid, 512, 0, s>>>(p);
        else if (mode == 1) dcn2_fwd_ws_kernel<T, IB, 1, true><<<grid, 512, 0, s>>>(p);
        else dcn2_fwd_ws_kernel<T, IB, 0, true><<<grid, 512, 0, s>>>(p);
    } else {
        if (mode == 2) dcn2_fwd_ws_kernel<T, IB, 2, false><<<grid, 512, 0, s>>>(p);
        else if (mode == 1) dcn2_fwd_ws_kernel<T, IB, 1, false><<<grid, 512, 0, s>>>(p);
        else dcn2_fwd_ws_kernel<T, IB, 0, false><<<grid, 512, 0, s>>>(p);
    }
    return hipGetLastError();
}

// The role election of dcn2_fwd_ws_kernel needs every SIMD to hold at most
// two waves of a workgroup, i.e. more than 512/3 VGPRs per wave.
template <typename T, int IB>
static bool ws_two_waves_per_simd() {
    static const bool ok = [] {
        const void *fns[6] = {reinterpret_cast<const void *>(&dcn2_fwd_ws_kernel<T, IB, 0, false>),
                              reinterpret_cast<const void *>(&dcn2_fwd_ws_kernel<T, IB, 1, false>),
                              reinterpret_cast<const void *>(&dcn2_fwd_ws_kernel<T, IB, 2, false>),
                              reinterpret_cast<const void *>(&dcn2_fwd_ws_kernel<T, IB, 0, true>),
                              reinterpret_cast<const void *>(&dcn2_fwd_ws_kernel<T, IB, 1, true>),
                              reinterpret_cast<const void *>(&dcn2_fwd_ws_kernel<T, IB, 2, true>)};
        for (const void *fn : fns) {
            hipFuncAttributes a;
            if (hipFuncGetAttributes(&a, fn) != hipSuccess || a.numRegs <= 512 / 3) return false;
        }
        return true;
    }();
    return ok;
}

// One launch over the output rows [row0, row0 + rows) with M tile bm (256 or
// 128 rows; rows and row0 are multiples of it).  fp32 (and 2-byte types with
// more than kBiasRows padded output rows): block tile 256x128 (8 waves of
// 32x128) when bm is 256, else 128x128 (8 waves of 64x32); both sample 128
// pixels, one slot per thread.
template <typename T>
static hipError_t launch_fwd_dt(const Geo &g, FwdParams p, int bm, int row0, int rows,
                                hipStream_t s) {
    p.mt_base = row0 / bm;
    p.mtiles = rows / bm;
    if constexpr (sizeof(T) == 2) {
        if (g.Mp <= kBiasRows) {
            if (bm == 256 && ws_two_waves_per_simd<T, 2>()) return launch_fwd_ws<T, 2>(g, p, s);
            if (bm == 128 && ws_two_waves_per_simd<T, 1>()) return launch_fwd_ws<T, 1>(g, p, s);
        }
        // more than kBiasRows output rows (or a register count that would let
        // three waves share a SIMD): the non-specialised kernel
        if (bm == 256) return launch_fwd_t<T, 8, 1, 1, 4>(g, p, s);
        return launch_fwd_t<T, 2, 4, 2, 1>(g, p, s);
    } else {
        if (bm == 256) return launch_fwd_t<T, 8, 1, 1, 4>(g, p, s);
        return launch_fwd_t<T, 2, 4, 2, 1>(g, p, s);
    }
}

// Ungrouped (or not splittable): one launch over every row and chunk.  With
// weight groups whose chunks never mix (Geo::gsplit): one launch per group
// over its Cout/WG rows and its cpw chunks per tap, so no launch samples or
// multiplies the zero blocks of the block-diagonal packed weight.
template <typename T>
static hipError_t launch_fwd_groups(const Geo &g, FwdParams p, hipStream_t s) {
    p.cpt = g.cpt;
    if (!g.gsplit) {
        p.cb = 0;
        p.cpw = g.cpt;
        p.nch_eff = g.Kp / g.KC;
        return launch_fwd_dt<T>(g, p, g.BM, 0, g.Mp, s);
    }
    const int cog = g.Cout / g.WG, bm = cog % 256 == 0 ? 256 : 128;
    p.cpw = g.cpw;
    p.nch_eff = g.KK * g.cpw;
    for (int w = 0; w < g.WG; ++w) {
        p.cb = w * g.cpw;
        const hipError_t e = launch_fwd_dt<T>(g, p, bm, w * cog, cog, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
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
    p.off_bs = g.off_bs;
    p.msk_bs = g.msk_bs;
    p.msk_logit = mask ? g.msk_logit : 0;
    p.bias = bias;
    p.out = out;
    p.out_nhwc = g.out_nhwc;
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
    p.Mp = g.Mp;
    switch (g.dtype) {
    case DCN2_F16: return launch_fwd_groups<f16>(g, p, s);
    case DCN2_BF16: return launch_fwd_groups<bf16>(g, p, s);
    default: return launch_fwd_groups<float>(g, p, s);
    }
}

}  // namespace dcn2
