// Fused DCNv2 forward for gfx950: bilinear, mask-modulated sampling into LDS
// feeding a 32x32 MFMA GEMM, never materialising the column matrix.
//
// Reference: im2colcuda + dcn_bilinear_cuda write columns[B][C*kh*kw][N] to
// HBM (com.cu:119-195), then gemm_cuda reads them back (com.cu:46-117).  Here
// one workgroup owns a BM x BN output tile (all of Cout when Cout <= 256) and
// walks K in chunks of KC channels of one (tap, group):
//
//   for chunk ch:                       (double-buffered LDS stage sB[2])
//     issue A (weight) fragment loads for ch+1      -- global/L2, 16 B per lane
//     compute descriptors + issue corner gathers for ch+1   -- channels-last xt
//     MFMA over sB[ch&1]                             -- matrix cores
//     finish the bilinear blend of ch+1 and store it to sB[(ch+1)&1]
//     barrier
//
// so the gathers and the blend of the next chunk overlap the MFMA of this one.
// Each sampled value is produced once per workgroup and reused by every output
// channel of the tile.
//
// Threads: 512 (8 waves) as WM x WN waves, each wave owning a 64x64 output
// sub-tile = 2x2 MFMA 32x32 blocks.  Sampling slot = (pixel, quarter of the
// chunk): 4 lanes cover one pixel's KC channels, so one corner of one pixel is
// read as a contiguous KC*sizeof(T)-byte run across 4 adjacent lanes.
#include "dcn2_common.h"
#include "dcn2_sampler.h"
#include "dcn2_kernels.h"
#include "../../include/dcnv2_amd.h"

namespace dcn2 {

struct FwdParams {
    const void *xt, *wp, *offset, *mask, *bias;
    void *out;
    int H, W, Cout, kh, kw, sh, sw, ph, pw, dh, dw, G, Cgp, Ho, Wo, Kp;
};

template <typename T, int WM, int WN>
__global__ __launch_bounds__(512) void dcn2_fwd_kernel(const FwdParams p) {
    using M = Mma<T>;
    using frag = typename M::frag;
    constexpr int KC = M::KC, KPL = M::KPL, KSTEP = M::KSTEP, NKS = KC / KSTEP;
    constexpr int BN = 64 * WN;
    constexpr int CPS = KC / 4;                 // channels per sampling slot
    constexpr int U4 = CPS * sizeof(T) / 16;    // 16-byte registers per corner per slot (2)
    constexpr int SPT = BN * 4 / 512;           // sampling slots per thread
    constexpr int LDK = KC + 16 / sizeof(T);    // LDS pitch (elements) of one pixel row
    static_assert(U4 == 2, "slot is 32 bytes per corner");

    __shared__ __attribute__((aligned(16))) T sB[2][BN][LDK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave - wm * WN;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * (64 * WM), b = blockIdx.z;
    const int N = p.Ho * p.Wo, KK = p.kh * p.kw, cs = p.G * p.Cgp;
    const int nch = KK * p.G * (p.Cgp / KC);

    const T *__restrict__ xt = (const T *)p.xt + (size_t)b * p.H * p.W * cs;
    const T *__restrict__ offs = (const T *)p.offset + (size_t)b * p.G * KK * 2 * N;
    const T *__restrict__ msk = p.mask ? (const T *)p.mask + (size_t)b * p.G * KK * N : nullptr;

    SampleGeo sg;
    sg.H = p.H; sg.W = p.W; sg.kh = p.kh; sg.kw = p.kw; sg.sh = p.sh; sg.sw = p.sw;
    sg.ph = p.ph; sg.pw = p.pw; sg.dh = p.dh; sg.dw = p.dw; sg.G = p.G; sg.Cgp = p.Cgp;
    sg.Wo = p.Wo; sg.N = N; sg.cs = cs; sg.KK = KK;
    Sampler<T, SPT> smp;
    smp.bind(n0, sg, tid);

    // Bilinear blend of the gathered corners, stored to LDS stage `buf` as
    // [pixel][channel] rows (the MFMA B-operand order).
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int s = 0; s < SPT; ++s) {
            const int pl = (tid + s * 512) >> 2;
            uint4 *dst = reinterpret_cast<uint4 *>(&sB[buf][pl][smp.q[s] * CPS]);
#pragma unroll
            for (int u = 0; u < U4; ++u) {
                float v[16 / sizeof(T)];
                smp.blend(s, u, v);
                dst[u] = pack16<T>(v);
            }
        }
    };

    // A (weight) fragments: rows m0 + wm*64 + i*32 + lane%32.
    const T *wrow[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
        wrow[i] = (const T *)p.wp + (size_t)(m0 + wm * 64 + i * 32 + (lane & 31)) * p.Kp +
                  (lane >> 5) * KPL;
    frag a_cur[2][NKS], a_nxt[2][NKS];
    auto load_a = [&](frag (&a)[2][NKS], int ch) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks)
                a[i][ks] = *reinterpret_cast<const frag *>(wrow[i] + ch * KC + ks * KSTEP);
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Prologue: chunk 0 into stage 0.
    load_a(a_cur, 0);
    smp.issue(0, sg, xt, offs, msk);
    store_stage(0);
    __syncthreads();

    for (int ch = 0; ch < nch; ++ch) {
        const int buf = ch & 1;
        const bool more = ch + 1 < nch;
        if (more) {
            load_a(a_nxt, ch + 1);
            smp.issue(ch + 1, sg, xt, offs, msk);
        }
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            frag bf[2];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = *reinterpret_cast<const frag *>(
                    &sB[buf][wn * 64 + j * 32 + (lane & 31)][ks * KSTEP + (lane >> 5) * KPL]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = M::mma(a_cur[i][ks], bf[j], acc[i][j]);
        }
        if (more) {
            store_stage(buf ^ 1);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) a_cur[i][ks] = a_nxt[i][ks];
        }
        __syncthreads();
    }

    // Epilogue: + bias, round to T, NCHW store.
    T *out = (T *)p.out + (size_t)b * p.Cout * N;
    const T *bias = (const T *)p.bias;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m >= p.Cout) continue;
            const float bv = bias ? to_f32(bias[m]) : 0.0f;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = n0 + wn * 64 + j * 32 + (lane & 31);
                if (n < N) out[(size_t)m * N + n] = from_f32<T>(acc[i][j][r] + bv);
            }
        }
    }
}

template <typename T, int WM, int WN>
static hipError_t launch_fwd_t(const Geo &g, const FwdParams &p, hipStream_t s) {
    dim3 grid(ceil_div(g.N, 64 * WN), g.Mp / (64 * WM), g.B);
    dcn2_fwd_kernel<T, WM, WN><<<grid, 512, 0, s>>>(p);
    return hipGetLastError();
}

template <typename T>
static hipError_t launch_fwd_dt(const Geo &g, const FwdParams &p, hipStream_t s) {
    if (g.BM == 256) return launch_fwd_t<T, 4, 2>(g, p, s);
    return launch_fwd_t<T, 2, 4>(g, p, s);
}

hipError_t launch_forward(const Geo &g, const void *xt, const void *wp, const void *offset,
                          const void *mask, const void *bias, void *out, hipStream_t s) {
    if (g.B == 0) return hipSuccess;
    FwdParams p;
    p.xt = xt;
    p.wp = wp;
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
