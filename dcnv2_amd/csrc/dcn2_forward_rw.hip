// Fused DCNv2 forward with the weight resident in registers, for the 3x3,
// <= 64-channel, 128 < Cout <= 256 fp16 shape class (the reference README's
// headline layer, README.md:14-19).
//
// Reference: im2colcuda + dcn_bilinear_cuda write the column matrix to HBM
// (com.cu:119-195) and gemm_cuda multiplies it with the weight (com.cu:46-117),
// re-reading the weight tile for every output tile.  Here the whole packed
// weight, 256 rows x 576 K in fp16 (288 KB), stays on chip for the life of the
// persistent workgroup: each of the four waves (one per SIMD, 512 registers)
// holds its 64 rows of taps 0-7 in its 256 AGPRs and tap 8 sits in LDS.  The
// loop then moves no weight bytes at all; the only vector-memory traffic is
// the corner gathers (32 KB per 64-pixel step), which is what bounds it.
//
// Input: the channels-last copy xt[b][y*W + x][64] of the pack kernel (or a
// channels-last input of 64 channels itself), so one bilinear corner of one
// pixel is one 128-byte run.  The blend multiplies the fp16 corner values by
// fp32 corner weights and sums in fp32 with v_fma_mix_f32 (one rounding of
// the blended column to fp16, as the reference samples in fp32 and rounds its
// columns, com.cu:119-148, 83, 87).  v_fma_mix issues between the MFMAs of
// the same wave almost for free; packed dot products do not (measured on
// MI355X: four v_dot2_f32_f16 per 32x32x16 MFMA double its time, four
// v_fma_mix_f32 add 15 %).  A corner outside the image has an offset past the
// image and reads zero from the buffer range check.
//
// Work: 64-pixel tiles of one image, all 256 output rows, walked persistently
// and XCD-aware.  One pipeline step per tap: the MFMAs of step s (16
// 32x32x16 per wave over LDS stage s % 3), the blend of step s+2 (gathered
// one step earlier) into its stage, the gathers of step s+3, one barrier; the
// first fragments of step s+1 are read before that barrier (their stage was
// completed a step earlier).  Each wave samples its own 16 pixels of every
// tap; their bilinear descriptors (four corner offsets and weights) are
// computed one tile ahead into an LDS ring that only that wave reads.
#include "dcn2_common.h"
#include "dcn2_kernels.h"
#include "../../include/dcnv2_amd.h"

namespace dcn2 {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

struct RwParams {
    const void *xt;      // channels-last input, 64 channels, one image = img_bytes
    const void *wp;      // fragment-ordered weight: 8 row blocks x 9 chunks x 4 k-steps
    const void *offset, *mask, *bias;
    void *out;
    int H, W, Wo, N, Cout, sh, sw, ph, pw, dh, dw;
    int ntiles, tiles;       // 64-pixel tiles per image, B * ntiles
    unsigned img_bytes;      // bytes of one image of xt: H*W*128
    unsigned out_img_bytes;  // Cout*N*2
    long long off_bs, msk_bs;
    int msk_logit;
};

constexpr int kRwPx = 64;     // pixels per tile
constexpr int kRwTaps = 9;    // K chunks (taps) per tile
constexpr int kRwLdk = 72;    // stage pitch (halfs): 144 bytes, conflict-free fragment reads


template <int MASK, bool ONHWC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void dcn2_fwd_rw_kernel(const RwParams p) {
    __shared__ __attribute__((aligned(16))) f16 stage[3][kRwPx][kRwLdk];
    // Descriptor ring, [tile parity][tap; 9 = sink for the idle lanes of the
    // last round][pixel]: the byte offsets of the four corners (y0,x0)
    // (y0,x0+1) (y0+1,x0) (y0+1,x0+1) inside the image (img_bytes outside it)
    // and their fp32 weights with the mask folded in.
    __shared__ __attribute__((aligned(16))) uint4 ringO[2][kRwTaps + 1][kRwPx];
    __shared__ __attribute__((aligned(16))) float4 ringW[2][kRwTaps + 1][kRwPx];
    // tap-8 weight fragments of every wave: [wave][ks*2 + rb][lane]
    __shared__ __attribute__((aligned(16))) f16x8 sA8[4][8][64];
    __shared__ __attribute__((aligned(16))) float sBias[256];
    // each wave's 64 x 64 output block on its way to HBM: [row][pixel] for an
    // NCHW output, [pixel][row] for a channels-last one
    __shared__ __attribute__((aligned(16))) f16 sOut[4][64][kRwLdk];

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int G = gridDim.x;
    const int my_tiles = (p.tiles - 1 - (int)blockIdx.x) / G + 1;  // grid <= tiles

    // ---------------------------------------------------------------- weights
    // Fragment (row block 2w + rb, chunk t, k-step ks) of the packed weight is
    // 64 lanes x 8 halfs at ((rb' * 9 + t) * 4 + ks) * 512 halfs.  Taps 0-7 go
    // straight into AGPRs (inline asm: the MFMAs then read them in place; a
    // compiler-visible load would land in VGPRs and be copied on every use).
    f16x8 aA[8][4][2];
    const f16 *wl = (const f16 *)p.wp + (size_t)lane * 8;
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                const f16 *src = wl + (size_t)(((2 * w + rb) * kRwTaps + t) * 4 + ks) * 512;
                asm volatile("global_load_dwordx4 %0, %1, off" : "=a"(aA[t][ks][rb]) : "v"(src));
            }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
            sA8[w][ks * 2 + rb][lane] = *reinterpret_cast<const f16x8 *>(
                wl + (size_t)(((2 * w + rb) * kRwTaps + 8) * 4 + ks) * 512);
    {
        const f16 *bias = (const f16 *)p.bias;
        const int m = w * 64 + lane;
        sBias[m] = (bias && m < p.Cout) ? (float)bias[m] : 0.0f;
    }

    // ---------------------------------------------------------------- tiles
    struct Tile {
        int b, n0;
        __amdgpu_buffer_rsrc_t xrs, ors;
        const f16 *offb, *mskb;
    };
    auto uni = [](int v) __attribute__((always_inline)) { return __builtin_amdgcn_readfirstlane(v); };
    auto tile_at = [&](int k) __attribute__((always_inline)) {
        Tile T;
        const int t = xcd_remap((int)blockIdx.x + min(k, my_tiles - 1) * G, p.tiles);
        T.b = uni(t / p.ntiles);
        T.n0 = uni((t - T.b * p.ntiles) * kRwPx);
        const char *xb = (const char *)p.xt + (size_t)T.b * p.img_bytes;
        T.xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(xb), (short)0, (int)p.img_bytes,
                                                  0x00020000);
        char *ob = (char *)p.out + (size_t)T.b * p.out_img_bytes;
        T.ors = __builtin_amdgcn_make_buffer_rsrc(ob, (short)0, (int)p.out_img_bytes, 0x00020000);
        T.offb = (const f16 *)p.offset + (size_t)T.b * p.off_bs;
        T.mskb = MASK ? (const f16 *)p.mask + (size_t)T.b * p.msk_bs : nullptr;
        return T;
    };

    // ---------------------------------------------------------------- descriptors
    // Lane l of wave w evaluates pixel P = 16w + l%16 of a tile for taps
    // 4r + l/16 in rounds r = 0, 1, 2 (taps past 8 write the sink row).
    const int dP = 16 * w + (lane & 15), dq = lane >> 4;
    struct OmRaw {
        int by, bx, live;
        f16 dy[3], dx[3], m[3];
    };
    auto load_om = [&](const Tile &T, OmRaw &o) __attribute__((always_inline)) {
        const int n = T.n0 + dP;
        o.live = n < p.N;
        const int nc = o.live ? n : p.N - 1;
        const int oy = nc / p.Wo, ox = nc - oy * p.Wo;
        o.by = oy * p.sh - p.ph;
        o.bx = ox * p.sw - p.pw;
#pragma unroll
        for (int r = 0; r < 3; ++r) {
            const int tap = min(4 * r + dq, kRwTaps - 1);
            o.dy[r] = T.offb[(size_t)(2 * tap) * p.N + nc];
            o.dx[r] = T.offb[(size_t)(2 * tap + 1) * p.N + nc];
            if constexpr (MASK) o.m[r] = T.mskb[(size_t)tap * p.N + nc];
        }
    };
    // One descriptor round in two halves, placed in different slices of a
    // step: the sample position (desc_pos) and the corner offsets, weights
    // and ring writes (desc_put).
    struct DescPos {
        int y0, x0;
        float ly, lx, mv;
    };
    auto desc_pos = [&](int r, const OmRaw &o) __attribute__((always_inline)) {
        const int tc = min(4 * r + dq, kRwTaps - 1);
        const int ki = (tc * 11) >> 5, kj = tc - 3 * ki;  // tc / 3, tc % 3 for tc < 9
        float y = (float)(o.by + ki * p.dh) + (float)o.dy[r];
        float x = (float)(o.bx + kj * p.dw) + (float)o.dx[r];
        // outside (-1,H)x(-1,W) everything samples 0; the clamp keeps the
        // float->int conversion defined for any learned offset
        y = fminf(fmaxf(y, -2.0f), (float)p.H + 1.0f);
        x = fminf(fmaxf(x, -2.0f), (float)p.W + 1.0f);
        const float fy = floorf(y), fx = floorf(x);
        DescPos d;
        d.y0 = (int)fy;
        d.x0 = (int)fx;
        d.ly = y - fy;
        d.lx = x - fx;
        float mv = 1.0f;
        if constexpr (MASK == 1) mv = (float)o.m[r];
        if constexpr (MASK == 2) mv = 1.0f / (1.0f + __expf(-(float)o.m[r]));
        d.mv = o.live ? mv : 0.0f;  // pixels past N sample 0
        return d;
    };
    auto desc_put = [&](int par, int r, const DescPos &d) __attribute__((always_inline)) {
        const int tap = 4 * r + dq;
        const float hy = 1.0f - d.ly, hx = 1.0f - d.lx;
        const float wy0 = hy * d.mv, wy1 = d.ly * d.mv;
        const int y0 = d.y0, x0 = d.x0;
        const bool vy0 = (unsigned)y0 < (unsigned)p.H, vy1 = (unsigned)(y0 + 1) < (unsigned)p.H;
        const bool vx0 = (unsigned)x0 < (unsigned)p.W, vx1 = (unsigned)(x0 + 1) < (unsigned)p.W;
        const unsigned base = (unsigned)(y0 * p.W + x0) * 128u, rowb = (unsigned)p.W * 128u;
        // (selects as bit masks: a conditional expression can become a
        // divergent branch that splits the step's scheduling region)
        auto pick = [&](bool v, unsigned o) __attribute__((always_inline)) {
            const unsigned m = 0u - (unsigned)v;
            return (o & m) | (p.img_bytes & ~m);
        };
        const int slot = tap < kRwTaps ? tap : kRwTaps;
        ringO[par][slot][dP] = make_uint4(pick(vy0 && vx0, base), pick(vy0 && vx1, base + 128u),
                                          pick(vy1 && vx0, base + rowb), pick(vy1 && vx1, base + rowb + 128u));
        ringW[par][slot][dP] = make_float4(wy0 * hx, wy0 * d.lx, wy1 * hx, wy1 * d.lx);
    };
    auto put_desc = [&](int par, int r, const OmRaw &o) __attribute__((always_inline)) {
        desc_put(par, r, desc_pos(r, o));
    };

    // ---------------------------------------------------------------- sampling
    // Lane l gathers 16-byte piece pc = l%8 (channels 8pc..8pc+7) of the four
    // corners of pixels 16w + 8i + pg, pg = l/8, i = 0, 1: 8 loads per step,
    // 8 lanes per 128-byte corner run.
    const int pc = lane & 7, pg = lane >> 3;
    uint4 gx[2][8];      // [set][4i + corner]
    // ring entries a step needs, read at its start: the corner offsets of the
    // gathers it issues and the corner weights of the pixels it blends
    auto ring_off = [&](uint4 (&ro)[2], int par, int tap) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; ++i) ro[i] = ringO[par][tap][16 * w + 8 * i + pg];
    };
    auto ring_wts = [&](float4 (&wt)[2], int par, int tap) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; ++i) wt[i] = ringW[par][tap][16 * w + 8 * i + pg];
    };
    // corners 2h, 2h+1 of pixel i
    auto gather2 = [&](auto set_c, const uint4 (&ro)[2], const Tile &T, auto i_c, auto h_c)
        __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value, i = decltype(i_c)::value, h = decltype(h_c)::value;
        const unsigned o[2] = {h ? ro[i].z : ro[i].x, h ? ro[i].w : ro[i].y};
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(T.xrs, (int)(o[q] + (unsigned)pc * 16u), 0, 0);
            gx[SET][4 * i + 2 * h + q] = make_uint4(v.x, v.y, v.z, v.w);
        }
    };
    auto gather = [&](auto set_c, const uint4 (&ro)[2], const Tile &T) __attribute__((always_inline)) {
        auto z = std::integral_constant<int, 0>{};
        auto o = std::integral_constant<int, 1>{};
        gather2(set_c, ro, T, z, z);
        gather2(set_c, ro, T, z, o);
        gather2(set_c, ro, T, o, z);
        gather2(set_c, ro, T, o, o);
    };
    // blend of channels 4h..4h+3 of pixel i from gather set SET: fp32
    // weights times fp16 corners, fp32 sums (v_fma_mix_f32)
    auto blend_half = [&](auto set_c, const float4 (&wt)[2], auto i_c, auto h_c, float (&v)[4])
        __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value, i = decltype(i_c)::value, h = decltype(h_c)::value;
        const float wq[4] = {wt[i].x, wt[i].y, wt[i].z, wt[i].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = 0.0f;
#pragma unroll
        for (int q = 3; q >= 0; --q) {  // the last-issued corner first: one wait covers all four
            const uint4 r = gx[SET][4 * i + q];
            const unsigned u[2] = {h ? r.z : r.x, h ? r.w : r.y};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const h2 x2 = __builtin_bit_cast(h2, u[c >> 1]);
                v[c] = fmaf(wq[q], (float)x2[c & 1], v[c]);
            }
        }
    };
    auto store_px = [&](int st, auto i_c, const float (&v0)[4], const float (&v1)[4])
        __attribute__((always_inline)) {
        constexpr int i = decltype(i_c)::value;
        typedef float f2 __attribute__((ext_vector_type(2)));
        const h2 a = __builtin_convertvector((f2){v0[0], v0[1]}, h2);
        const h2 b = __builtin_convertvector((f2){v0[2], v0[3]}, h2);
        const h2 c = __builtin_convertvector((f2){v1[0], v1[1]}, h2);
        const h2 d = __builtin_convertvector((f2){v1[2], v1[3]}, h2);
        *reinterpret_cast<u32x4 *>(&stage[st][16 * w + 8 * i + pg][8 * pc]) =
            u32x4{__builtin_bit_cast(unsigned, a), __builtin_bit_cast(unsigned, b),
                  __builtin_bit_cast(unsigned, c), __builtin_bit_cast(unsigned, d)};
    };
    auto blend = [&](auto set_c, int st, int par, int tap) __attribute__((always_inline)) {
        float4 wt[2];
        ring_wts(wt, par, tap);
        float v0[4], v1[4];
        blend_half(set_c, wt, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, v0);
        blend_half(set_c, wt, std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{}, v1);
        store_px(st, std::integral_constant<int, 0>{}, v0, v1);
        blend_half(set_c, wt, std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{}, v0);
        blend_half(set_c, wt, std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{}, v1);
        store_px(st, std::integral_constant<int, 1>{}, v0, v1);
    };
    auto gather_at = [&](auto set_c, int par, int tap, const Tile &T) __attribute__((always_inline)) {
        uint4 ro[2];
        ring_off(ro, par, tap);
        gather(set_c, ro, T);
    };

    // ---------------------------------------------------------------- MFMA
    f32x16 acc[2][2];
    const int mrow = w * 64 + (lane & 31);  // NCHW: output row of this lane in row block rb: mrow + 32 rb
    float bias_r[2];
    auto init_acc = [&]() __attribute__((always_inline)) {
        if constexpr (ONHWC) {
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const f32x4 b4 = *reinterpret_cast<const f32x4 *>(
                        &sBias[w * 64 + rb * 32 + 8 * q + 4 * (lane >> 5)]);
#pragma unroll
                    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[rb][pb][4 * q + e] = b4[e];
                }
        } else {
            typedef unsigned long long u64x8 __attribute__((ext_vector_type(8)));
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                // (the empty asm keeps the compiler from hoisting the 32-register
                // bias image out of the loop and holding it for the whole kernel)
                float br = bias_r[rb];
                asm volatile("" : "+v"(br));
                const uint32_t bb = __float_as_uint(br);
                const unsigned long long b2 = ((unsigned long long)bb << 32) | bb;
#pragma unroll
                for (int pb = 0; pb < 2; ++pb) acc[rb][pb] = __builtin_bit_cast(f32x16, u64x8(b2));
            }
        }
    };
    // B fragments (the sampled columns) of k-step ks of LDS stage st
    auto read_bf = [&](f16x8 (&bf)[2], int st, int ks) __attribute__((always_inline)) {
#pragma unroll
        for (int pb = 0; pb < 2; ++pb)
            bf[pb] = *reinterpret_cast<const f16x8 *>(
                &stage[st][pb * 32 + (lane & 31)][ks * 16 + (lane >> 5) * 8]);
    };
    auto mfma_ks = [&](auto tap_c, auto ks_c, const f16x8 (&bf)[2]) __attribute__((always_inline)) {
        constexpr int TAP = decltype(tap_c)::value, ks = decltype(ks_c)::value;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            f16x8 a;
            if constexpr (TAP < 8) a = aA[TAP][ks][rb];
            else a = sA8[w][ks * 2 + rb][lane];
#pragma unroll
            for (int pb = 0; pb < 2; ++pb) {
                if constexpr (ONHWC)
                    acc[rb][pb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bf[pb], acc[rb][pb], 0, 0, 0);
                else
                    acc[rb][pb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[pb], a, acc[rb][pb], 0, 0, 0);
            }
        }
    };
    // Output of a tile: the accumulators are rounded to fp16 and staged in
    // this wave's LDS block at the tile's last step (stage_out: 4 consecutive
    // pixels of one row, NCHW, or 4 consecutive channels of one pixel,
    // channels-last, per 8-byte write); during the next tile's first step the
    // block is read back and written as 16-byte pieces, 8 lanes per 128-byte
    // run of a row (or a pixel), two store instructions per slice (flush_out),
    // so every store covers 8 whole 128-byte lines and no step waits for the
    // LDS round trip.  Pieces outside the output get an offset past the buffer
    // and are dropped (N % 8 == 0, resp. Cout % 8 == 0: a piece is all in or
    // all out).
    auto stage_out = [&]() __attribute__((always_inline)) {
        f16(&so)[64][kRwLdk] = sOut[w];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int pb = 0; pb < 2; ++pb)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    typedef float f2 __attribute__((ext_vector_type(2)));
                    const h2 lo = __builtin_convertvector((f2){acc[rb][pb][4 * q], acc[rb][pb][4 * q + 1]}, h2);
                    const h2 hi = __builtin_convertvector((f2){acc[rb][pb][4 * q + 2], acc[rb][pb][4 * q + 3]}, h2);
                    f16 *dst;
                    if constexpr (ONHWC)
                        dst = &so[pb * 32 + (lane & 31)][rb * 32 + 8 * q + 4 * (lane >> 5)];
                    else
                        dst = &so[rb * 32 + (lane & 31)][pb * 32 + 8 * q + 4 * (lane >> 5)];
                    *reinterpret_cast<u32x2 *>(dst) =
                        u32x2{__builtin_bit_cast(unsigned, lo), __builtin_bit_cast(unsigned, hi)};
                }
    };
    auto flush_out = [&](const Tile &T, int it0) __attribute__((always_inline)) {
        f16(&so)[64][kRwLdk] = sOut[w];
        const int seg = lane & 7;
        uint4 v[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) v[k] = *reinterpret_cast<const uint4 *>(&so[(it0 + k) * 8 + (lane >> 3)][seg * 8]);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int row = (it0 + k) * 8 + (lane >> 3);
            unsigned off;
            if constexpr (ONHWC) {
                const int n = T.n0 + row, m = w * 64 + seg * 8;
                off = (n < p.N && m < p.Cout) ? ((unsigned)n * (unsigned)p.Cout + (unsigned)m) * 2u
                                              : p.out_img_bytes;
            } else {
                const int m = w * 64 + row, n = T.n0 + seg * 8;
                off = (n < p.N && m < p.Cout) ? ((unsigned)m * (unsigned)p.N + (unsigned)n) * 2u
                                              : p.out_img_bytes;
            }
            // non-temporal: the output is not read again by this kernel, so
            // its lines should not push the gathered input out of the L2
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{v[k].x, v[k].y, v[k].z, v[k].w}, T.ors, (int)off, 0, 2);
        }
    };

    // ---------------------------------------------------------------- prologue
    Tile cur = tile_at(0), nxt = tile_at(1);
    // the "previous tile" of the first one: an output buffer of no records,
    // so its flush stores are dropped
    Tile prv = cur;
    prv.ors = __builtin_amdgcn_make_buffer_rsrc(p.out, (short)0, 0, 0x00020000);
    OmRaw om;
    load_om(cur, om);
    __syncthreads();  // sA8 and sBias written
    if constexpr (!ONHWC) {
        const f16 *bias = (const f16 *)p.bias;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) bias_r[rb] = sBias[mrow + rb * 32];
        (void)bias;
    }
#pragma unroll
    for (int r = 0; r < 3; ++r) put_desc(0, r, om);
    load_om(nxt, om);  // tile 1's offsets, turned into descriptors during tile 0
    // the tap-0..7 weights are complete once every earlier vector load is
    // (loads return in order); tie the AGPRs to that wait
#pragma unroll
    for (int t = 0; t < 8; ++t)
        asm volatile("s_waitcnt vmcnt(0)"
                     : "+a"(aA[t][0][0]), "+a"(aA[t][0][1]), "+a"(aA[t][1][0]), "+a"(aA[t][1][1]),
                       "+a"(aA[t][2][0]), "+a"(aA[t][2][1]), "+a"(aA[t][3][0]), "+a"(aA[t][3][1]));
    gather_at(std::integral_constant<int, 0>{}, 0, 0, cur);
    gather_at(std::integral_constant<int, 1>{}, 0, 1, cur);
    blend(std::integral_constant<int, 0>{}, 0, 0, 0);
    gather_at(std::integral_constant<int, 0>{}, 0, 2, cur);
    blend(std::integral_constant<int, 1>{}, 1, 0, 1);
    init_acc();
    __syncthreads();
    // fragments of the first two k-steps of the next step, read ahead of the
    // barrier that starts it (its stage was completed one step earlier)
    f16x8 bfA[2], bfB[2];
    read_bf(bfA, 0, 0);
    read_bf(bfB, 0, 1);

    // ---------------------------------------------------------------- main loop
    // Tile k, tap J is global step s = 9k + J.  Its columns are gathered in
    // step s-3 into register set s % 2, blended in step s-2 into LDS stage
    // s % 3 and multiplied in step s; descriptor ring k % 2.  With P = k % 2
    // all of these are compile-time constants inside tile<P> (9 % 3 == 0).
    auto tile = [&](auto p_c) __attribute__((always_inline)) {
        constexpr int P = decltype(p_c)::value;
        auto step = [&](auto j_c) __attribute__((always_inline)) {
            constexpr int J = decltype(j_c)::value;
            constexpr int SM = J % 3, SB = (J + 2) % 3, SN = (J + 1) % 3;  // stages
            constexpr int GB = (P + J) & 1, GI = GB ^ 1;                    // gather sets
            // step s+3 (gathered now) and s+2 (blended now): tap and ring
            constexpr int IT = J + 3 < kRwTaps ? J + 3 : J + 3 - kRwTaps;
            constexpr int IP = J + 3 < kRwTaps ? P : P ^ 1;
            constexpr int BT = J + 2 < kRwTaps ? J + 2 : J + 2 - kRwTaps;
            constexpr int BP = J + 2 < kRwTaps ? P : P ^ 1;
            // The step runs in four slices, one per k-step, fenced so that the
            // compiler keeps this interleave: the k-step's 4 MFMAs (128
            // cycles of the matrix core) with the fragment reads of a later
            // k-step and about 24 other instructions, i.e. what one wave can
            // issue while its MFMAs run.  Slice 0 issues the gathers of step
            // s+3; slices 1-3 blend the four pixel groups of step s+2.
            auto set_b = std::integral_constant<int, GB>{};
            auto i0_c = std::integral_constant<int, 0>{};
            auto i1_c = std::integral_constant<int, 1>{};
            uint4 ro[2];
            float4 wt[2];
            float v0[4], v1[4];
            // gathers of step s+3 go out two per slice (pixel 0 in slices 0-1,
            // pixel 1 in slices 2-3), so the wave never blocks on a full
            // vector-memory queue for a whole batch; each pixel's loads still
            // have a full step before its blend (pixel 0 in slice 1, pixel 1
            // in slices 2-3 of the next step)
            const Tile &TI = J + 3 < kRwTaps ? cur : nxt;
            auto set_i = std::integral_constant<int, GI>{};
            // descriptor round J-2 of the next tile (steps 2-4): position in
            // slice 1, offsets / weights / ring writes in slice 3
            constexpr bool DESC = J >= 2 && J <= 4;
            DescPos dpos;
            ring_off(ro, IP, IT);
            ring_wts(wt, BP, BT);
            __builtin_amdgcn_sched_barrier(0);
            mfma_ks(std::integral_constant<int, J>{}, std::integral_constant<int, 0>{}, bfA);
            gather2(set_i, ro, TI, i0_c, i0_c);
            read_bf(bfA, SM, 2);
            if constexpr (J == 0) flush_out(prv, 0);
            __builtin_amdgcn_sched_barrier(0);
            mfma_ks(std::integral_constant<int, J>{}, std::integral_constant<int, 1>{}, bfB);
            gather2(set_i, ro, TI, i0_c, i1_c);
            blend_half(set_b, wt, i0_c, i0_c, v0);
            blend_half(set_b, wt, i0_c, i1_c, v1);
            store_px(SB, i0_c, v0, v1);
            read_bf(bfB, SM, 3);
            if constexpr (J == 0) flush_out(prv, 2);
            if constexpr (DESC) dpos = desc_pos(J - 2, om);
            __builtin_amdgcn_sched_barrier(0);
            mfma_ks(std::integral_constant<int, J>{}, std::integral_constant<int, 2>{}, bfA);
            gather2(set_i, ro, TI, i1_c, i0_c);
            blend_half(set_b, wt, i1_c, i0_c, v0);
            read_bf(bfA, SN, 0);
            if constexpr (J == 0) flush_out(prv, 4);
            __builtin_amdgcn_sched_barrier(0);
            mfma_ks(std::integral_constant<int, J>{}, std::integral_constant<int, 3>{}, bfB);
            gather2(set_i, ro, TI, i1_c, i1_c);
            blend_half(set_b, wt, i1_c, i1_c, v1);
            store_px(SB, i1_c, v0, v1);
            read_bf(bfB, SN, 1);
            if constexpr (J == 0) flush_out(prv, 6);
            if constexpr (DESC) desc_put(P ^ 1, J - 2, dpos);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (J == kRwTaps - 1) {
                stage_out();
                init_acc();
            }
            __syncthreads();
        };
        step(std::integral_constant<int, 0>{});
        step(std::integral_constant<int, 1>{});
        step(std::integral_constant<int, 2>{});
        step(std::integral_constant<int, 3>{});
        step(std::integral_constant<int, 4>{});
        step(std::integral_constant<int, 5>{});
        step(std::integral_constant<int, 6>{});
        step(std::integral_constant<int, 7>{});
        step(std::integral_constant<int, 8>{});
    };
    int k = 0;
    for (; k + 2 <= my_tiles; k += 2) {
        tile(std::integral_constant<int, 0>{});
        prv = cur;
        cur = nxt;
        nxt = tile_at(k + 2);
        load_om(nxt, om);
        tile(std::integral_constant<int, 1>{});
        prv = cur;
        cur = nxt;
        nxt = tile_at(k + 3);
        load_om(nxt, om);
    }
    if (k < my_tiles) {
        tile(std::integral_constant<int, 0>{});
        prv = cur;
    }
    // the last tile's output (staged at its last step)
#pragma unroll
    for (int it = 0; it < 8; it += 2) flush_out(prv, it);
}

bool rw_eligible(const Geo &g) {
    return g.dtype == DCN2_F16 && g.G == 1 && g.Cgp == 64 && g.KK == kRwTaps && g.Mp == 256 &&
           g.WG == 1 && (g.out_nhwc ? g.Cout % 8 == 0 : g.N % 8 == 0) &&
           (long long)g.Cout * g.N * 2 < 0x7fffffffLL;
}

hipError_t launch_forward_rw(const Geo &g, const void *xt, const void *wp, const void *offset,
                             const void *mask, const void *bias, void *out, hipStream_t s) {
    if (g.B == 0) return hipSuccess;
    RwParams p;
    p.xt = xt;
    p.wp = wp;
    p.offset = offset;
    p.mask = mask;
    p.bias = bias;
    p.out = out;
    p.H = g.H;
    p.W = g.W;
    p.Wo = g.Wo;
    p.N = g.N;
    p.Cout = g.Cout;
    p.sh = g.sh;
    p.sw = g.sw;
    p.ph = g.ph;
    p.pw = g.pw;
    p.dh = g.dh;
    p.dw = g.dw;
    p.ntiles = ceil_div(g.N, kRwPx);
    p.tiles = g.B * p.ntiles;
    p.img_bytes = (unsigned)((size_t)g.H * g.W * 128);
    p.out_img_bytes = (unsigned)((size_t)g.Cout * g.N * 2);
    p.off_bs = g.off_bs;
    p.msk_bs = g.msk_bs;
    p.msk_logit = mask ? g.msk_logit : 0;
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
        ncu = 256;
    const int grid = p.tiles < ncu ? p.tiles : ncu;
    const int mode = mask ? (p.msk_logit ? 2 : 1) : 0;
    if (g.out_nhwc) {
        if (mode == 2) dcn2_fwd_rw_kernel<2, true><<<grid, 256, 0, s>>>(p);
        else if (mode == 1) dcn2_fwd_rw_kernel<1, true><<<grid, 256, 0, s>>>(p);
        else dcn2_fwd_rw_kernel<0, true><<<grid, 256, 0, s>>>(p);
    } else {
        if (mode == 2) dcn2_fwd_rw_kernel<2, false><<<grid, 256, 0, s>>>(p);
        else if (mode == 1) dcn2_fwd_rw_kernel<1, false><<<grid, 256, 0, s>>>(p);
        else dcn2_fwd_rw_kernel<0, false><<<grid, 256, 0, s>>>(p);
    }
    return hipGetLastError();
}

}  // namespace dcn2
