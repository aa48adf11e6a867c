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
// Input layout (pack_input_pairs in dcn2_pack.hip): xp[b][yy][j][c][2] with
// yy = y + 1 in [0, H+2) and j in [0, W]: the channel-c value of pixels
// (y, j-1) and (y, j) side by side (zero outside the image, and rows yy = 0
// and H+1 all zero).  A bilinear sample at (y0 + ly, x0 + lx) then reads two
// 256-byte runs, row yy = y0+1 and row yy+1 at pair j = x0+1, and each 32-bit
// word is the (left, right) corner pair of one channel: the blend is two
// v_dot2_f32_f16 per channel, (w00, w01).(x00, x01) + (w10, w11).(x10, x11),
// with exact products and fp32 sums.  The corner weights are rounded to fp16
// for the dot products (relative 2^-12); the blended column is rounded once to
// fp16 for the MFMA, as the reference rounds its columns (com.cu:83, 87).
// Corners outside the image read the stored zeros, and a sample with no
// corner inside reads past the image (zeros from the buffer range check).
//
// Work: 64-pixel tiles of one image, all 256 output rows, walked persistently
// and XCD-aware.  One pipeline step per tap: the MFMAs of tap t (16 32x32x16
// per wave over the LDS stage of t), the blend of tap t+1 (gathered one step
// earlier) into the other stage, the gathers of tap t+2, one barrier.  Each
// wave samples its own 16 pixels of every tap; their bilinear descriptors
// (row offset, two weight pairs) are computed one tile ahead into an LDS ring
// that only that wave reads.
#include "dcn2_common.h"
#include "dcn2_kernels.h"
#include "../../include/dcnv2_amd.h"

namespace dcn2 {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

struct RwParams {
    const void *xp;      // pair-packed input, one image = img_bytes
    const void *wp;      // fragment-ordered weight: 8 row blocks x 9 chunks x 4 k-steps
    const void *offset, *mask, *bias;
    void *out;
    int H, W, Wo, N, Cout, sh, sw, ph, pw, dh, dw;
    int ntiles, tiles;       // 64-pixel tiles per image, B * ntiles
    unsigned img_bytes;      // bytes of one image of xp: (H+2)*(W+1)*256
    unsigned row_bytes;      // (W+1)*256
    unsigned out_img_bytes;  // Cout*N*2
    long long off_bs, msk_bs;
    int msk_logit;
};

constexpr int kRwPx = 64;     // pixels per tile
constexpr int kRwTaps = 9;    // K chunks (taps) per tile
constexpr int kRwLdk = 72;    // stage pitch (halfs): 144 bytes, conflict-free fragment reads

// Descriptor of one (tap, pixel) in the ring: x = byte offset of the sample's
// first row pair inside the image of xp (img_bytes: no corner inside),
// y = fp16 weights (w00, w01) of that row, z = (w10, w11) of the next row.
typedef uint4 RwDesc;

template <int MASK, bool ONHWC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void dcn2_fwd_rw_kernel(const RwParams p) {
    __shared__ __attribute__((aligned(16))) f16 stage[3][kRwPx][kRwLdk];
    // [tile parity][tap; 9 = sink for the idle lanes of the last round][pixel]
    __shared__ __attribute__((aligned(16))) RwDesc ring[2][kRwTaps + 1][kRwPx];
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
        const char *xb = (const char *)p.xp + (size_t)T.b * p.img_bytes;
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
    auto put_desc = [&](int par, int r, const OmRaw &o) __attribute__((always_inline)) {
        const int tap = 4 * r + dq;
        const int tc = min(tap, kRwTaps - 1);
        const int ki = (tc * 11) >> 5, kj = tc - 3 * ki;  // tc / 3, tc % 3 for tc < 9
        float y = (float)(o.by + ki * p.dh) + (float)o.dy[r];
        float x = (float)(o.bx + kj * p.dw) + (float)o.dx[r];
        // outside (-1,H)x(-1,W) everything samples 0; the clamp keeps the
        // float->int conversion defined for any learned offset
        y = fminf(fmaxf(y, -2.0f), (float)p.H + 1.0f);
        x = fminf(fmaxf(x, -2.0f), (float)p.W + 1.0f);
        const float fy = floorf(y), fx = floorf(x);
        const int y0 = (int)fy, x0 = (int)fx;
        const float ly = y - fy, lx = x - fx, hy = 1.0f - ly, hx = 1.0f - lx;
        float mv = 1.0f;
        if constexpr (MASK == 1) mv = (float)o.m[r];
        if constexpr (MASK == 2) mv = 1.0f / (1.0f + __expf(-(float)o.m[r]));
        mv = o.live ? mv : 0.0f;  // pixels past N sample 0
        const float wy0 = hy * mv, wy1 = ly * mv;
        const h2 w0 = __builtin_convertvector((float __attribute__((ext_vector_type(2)))){wy0 * hx, wy0 * lx}, h2);
        const h2 w1 = __builtin_convertvector((float __attribute__((ext_vector_type(2)))){wy1 * hx, wy1 * lx}, h2);
        // some corner inside: y0 in [-1, H-1] and x0 in [-1, W-1]
        const bool in = (unsigned)(y0 + 1) <= (unsigned)p.H && (unsigned)(x0 + 1) <= (unsigned)p.W;
        const unsigned off = (unsigned)((y0 + 1) * (p.W + 1) + (x0 + 1)) * 256u;
        RwDesc d;
        d.x = in ? off : p.img_bytes;
        d.y = __builtin_bit_cast(unsigned, w0);
        d.z = __builtin_bit_cast(unsigned, w1);
        d.w = 0;
        ring[par][tap < kRwTaps ? tap : kRwTaps][dP] = d;
    };

    // ---------------------------------------------------------------- sampling
    // Lane l gathers 16-byte piece pc = l%16 (channels 4pc..4pc+3, both
    // pixels of the pair) of pixels 16w + 4i + sq, i = 0..3, rows 0 and 1.
    const int pc = lane & 15, sq = lane >> 4;
    uint4 gx[2][8];      // [set][2i + row]
    // ring entries a step needs, read at its start: the row offsets of the
    // gathers it issues and the weight pairs of the pixels it blends
    auto ring_off = [&](unsigned (&ro)[4], int par, int tap) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ro[i] = ring[par][tap][16 * w + 4 * i + sq].x;
    };
    auto ring_wts = [&](uint2 (&wt)[4], int par, int tap) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const RwDesc d = ring[par][tap][16 * w + 4 * i + sq];
            wt[i] = make_uint2(d.y, d.z);
        }
    };
    auto gather = [&](auto set_c, const unsigned (&ro)[4], const Tile &T) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int voff = (int)(ro[i] + (unsigned)pc * 16u);
            const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(T.xrs, voff, 0, 0);
            const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(T.xrs, voff, (int)p.row_bytes, 0);
            gx[SET][2 * i] = make_uint4(v0.x, v0.y, v0.z, v0.w);
            gx[SET][2 * i + 1] = make_uint4(v1.x, v1.y, v1.z, v1.w);
        }
    };
    // blend of the data gathered into set SET for ring entry (par, tap):
    // the weight pairs are read back from the ring (still intact: a tile's
    // entries are only replaced in the middle of the next tile)
    auto blend_px = [&](auto set_c, int st, const uint2 (&wt)[4], auto i_c) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value;
        {
            constexpr int i = decltype(i_c)::value;
            const uint4 r0 = gx[SET][2 * i], r1 = gx[SET][2 * i + 1];
            const uint2 d = make_uint2(wt[i].x, wt[i].y);
            const h2 w1 = __builtin_bit_cast(h2, d.y);
            const unsigned a0[4] = {r0.x, r0.y, r0.z, r0.w}, a1[4] = {r1.x, r1.y, r1.z, r1.w};
            float v[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                // first product pair with the VOP3P form and a zero addend (the
                // accumulating VOP2 form would need a zeroing move first)
                asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(v[c]) : "v"(a0[c]), "v"(d.x));
                v[c] = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a1[c]), w1, v[c], false);
            }
            typedef float f2 __attribute__((ext_vector_type(2)));
            const h2 lo = __builtin_convertvector((f2){v[0], v[1]}, h2);
            const h2 hi = __builtin_convertvector((f2){v[2], v[3]}, h2);
            *reinterpret_cast<u32x2 *>(&stage[st][16 * w + 4 * i + sq][4 * pc]) =
                u32x2{__builtin_bit_cast(unsigned, lo), __builtin_bit_cast(unsigned, hi)};
        }
    };
    auto blend = [&](auto set_c, int st, int par, int tap) __attribute__((always_inline)) {
        uint2 wt[4];
        ring_wts(wt, par, tap);
        blend_px(set_c, st, wt, std::integral_constant<int, 0>{});
        blend_px(set_c, st, wt, std::integral_constant<int, 1>{});
        blend_px(set_c, st, wt, std::integral_constant<int, 2>{});
        blend_px(set_c, st, wt, std::integral_constant<int, 3>{});
    };
    auto gather_at = [&](auto set_c, int par, int tap, const Tile &T) __attribute__((always_inline)) {
        unsigned ro[4];
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
                const uint32_t bb = __float_as_uint(bias_r[rb]);
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
    // Output of the tile: the accumulators are rounded to fp16 and staged in
    // this wave's LDS block (4 consecutive pixels of one row, NCHW, or 4
    // consecutive channels of one pixel, channels-last, per 8-byte write),
    // then written as 16-byte pieces, 8 lanes per 128-byte run of a row (or a
    // pixel), so every store instruction covers 8 whole 128-byte lines.
    // Pieces outside the output get an offset past the buffer and are dropped
    // (N % 8 == 0, resp. Cout % 8 == 0: a piece is all in or all out).
    auto store_tile = [&](const Tile &T) __attribute__((always_inline)) {
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
        const int seg = lane & 7;
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            const int row = it * 8 + (lane >> 3);
            const uint4 v = *reinterpret_cast<const uint4 *>(&so[row][seg * 8]);
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
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{v.x, v.y, v.z, v.w}, T.ors, (int)off, 0, 2);
        }
    };

    // ---------------------------------------------------------------- prologue
    Tile cur = tile_at(0), nxt = tile_at(1);
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
            unsigned ro[4];
            uint2 wt[4];
            ring_off(ro, IP, IT);
            ring_wts(wt, BP, BT);
            __builtin_amdgcn_sched_barrier(0);
            mfma_ks(std::integral_constant<int, J>{}, std::integral_constant<int, 0>{}, bfA);
            gather(std::integral_constant<int, GI>{}, ro, J + 3 < kRwTaps ? cur : nxt);
            read_bf(bfA, SM, 2);
            __builtin_amdgcn_sched_barrier(0);
            mfma_ks(std::integral_constant<int, J>{}, std::integral_constant<int, 1>{}, bfB);
            blend_px(set_b, SB, wt, std::integral_constant<int, 0>{});
            blend_px(set_b, SB, wt, std::integral_constant<int, 1>{});
            read_bf(bfB, SM, 3);
            __builtin_amdgcn_sched_barrier(0);
            mfma_ks(std::integral_constant<int, J>{}, std::integral_constant<int, 2>{}, bfA);
            blend_px(set_b, SB, wt, std::integral_constant<int, 2>{});
            read_bf(bfA, SN, 0);
            __builtin_amdgcn_sched_barrier(0);
            mfma_ks(std::integral_constant<int, J>{}, std::integral_constant<int, 3>{}, bfB);
            blend_px(set_b, SB, wt, std::integral_constant<int, 3>{});
            read_bf(bfB, SN, 1);
            if constexpr (J >= 2 && J <= 4) put_desc(P ^ 1, J - 2, om);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (J == kRwTaps - 1) {
                store_tile(cur);
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
        cur = nxt;
        nxt = tile_at(k + 2);
        load_om(nxt, om);
        tile(std::integral_constant<int, 1>{});
        cur = nxt;
        nxt = tile_at(k + 3);
        load_om(nxt, om);
    }
    if (k < my_tiles) tile(std::integral_constant<int, 0>{});
}

bool rw_eligible(const Geo &g) {
    return g.dtype == DCN2_F16 && g.G == 1 && g.Cgp == 64 && g.KK == kRwTaps && g.Mp == 256 &&
           g.WG == 1 && (g.out_nhwc ? g.Cout % 8 == 0 : g.N % 8 == 0) &&
           (long long)(g.H + 2) * (g.W + 1) * 256 < 0x7fffffffLL &&
           (long long)g.Cout * g.N * 2 < 0x7fffffffLL;
}

size_t rw_input_bytes(const Geo &g) { return (size_t)g.B * (g.H + 2) * (g.W + 1) * 256; }

hipError_t launch_forward_rw(const Geo &g, const void *xp, const void *wp, const void *offset,
                             const void *mask, const void *bias, void *out, hipStream_t s) {
    if (g.B == 0) return hipSuccess;
    RwParams p;
    p.xp = xp;
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
    p.img_bytes = (unsigned)((size_t)(g.H + 2) * (g.W + 1) * 256);
    p.row_bytes = (unsigned)((g.W + 1) * 256);
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
