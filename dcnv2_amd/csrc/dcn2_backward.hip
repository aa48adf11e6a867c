// DCNv2 backward for gfx950.
//
// Reference (com.cu:733-848) loops over the batch on the host and, per image,
// runs a cuBLAS GEMM for the column gradient (com.cu:789-793), the coordinate
// kernel (com.cu:431-501), the col2im atomic scatter (com.cu:553-609), a
// second im2col (com.cu:637-706) and two more cuBLAS calls for grad_weight and
// grad_bias (com.cu:829-835).  Here the whole batch is one launch per stage:
//
//  bucket passes   each sample (image, offset plane, pixel) gets a row in the
//                  bucket of the 16x16 cell tile its bilinear cell lies in
//                  (count, scan, place; the rows are sized exactly)
//  fused kernel    (2-byte types, 128 < Cout <= 256, one K chunk per group)
//     cg[k][n] = sum_m Wt[k][m] * gO[m][n]            MFMA, kept on chip (LDS)
//     grad_mask / grad_offset  via the corner sums    S_q = sum_c cg_c * x_c(corner q)
//         grad_mask = sum_q w_q S_q,  grad_off_y = mask * sum_q dw_q/dy S_q, ...
//       (4 multiply-adds per channel instead of re-evaluating bilinear and
//        both coordinate weights per channel as com.cu:486-492 does)
//     the masked cg row of each sample -> its bucket row
//     gW[m][k] += sum_n gO[m][n] * col[k][n]           MFMA over the columns
//       blended from the same corner gathers; grad_bias from the same gO
//  otherwise       dcn2_colgrad_kernel (all but grad_weight) and a grad_weight
//                  kernel that re-samples the columns
//  grad_input      per cell tile, from the tile's bucket rows (no atomics):
//                  summed by cells or pulled per pixel, written straight to
//                  grad_input in the caller's type and layout; then the
//                  tile-boundary pixels from the tiles' border rings (and
//                  grad_weight / grad_bias in the same launch).
#include <algorithm>
#include <cstddef>
#include <cstdlib>
#include <type_traits>

#include "dcn2_common.h"
#include "dcn2_sampler.h"
#include "dcn2_kernels.h"
#include "dcn2_profile.h"
#include "../../include/dcnv2_amd.h"

namespace dcn2 {

// Record of a placed sample: its floor corner (y0 in the low, x0 in the high
// 16 bits, both >= -2) and the bilinear fractions (12 bytes: the consumers
// find the sample's hand-off row from the record's own position).
struct BucketRec {
    int yx;
    float ly, lx;
};

struct BwdParams {
    const void *xt, *wt, *tab, *offset, *mask, *gout;
    void *goff, *gmask;
    float *gi_acc, *gw_acc, *gb_acc;
    int B, H, W, Cout, kh, kw, sh, sw, ph, pw, dh, dw, G, Cg, Cgp, Ho, Wo, Kp, Mp;
    int tiles_per_img, splits;
    int go_nhwc;  // grad_output is channels-last [B][Ho][Wo][Cout]
    // grad_output can be read with 16-byte loads: 8 consecutive pixels of a row
    // (NCHW, N % 8 == 0) or channels of a pixel (channels-last, Cout % 8 == 0),
    // from a 16-byte aligned base
    int go_vec;
    // grad_input gather: cell-tile buckets (see dcn2_gi_gather_kernel).  The
    // rows of all buckets are packed back to back, bucket k owning rows
    // [bstart[k], bstart[k+1]); there are at most B*G*KK*N of them (one per
    // sample), so the storage is sized exactly and no bucket can overflow.
    void *cgm;          // [rows][Cgp] masked column gradient rows (RowOf)
    unsigned char *rsc; // [rows][Cgp/32] scale codes of bf16 rows (row_block_scale)
    float *csum;        // [B][G*KK][N][4] corner sums of groups of several chunks (fused kernel)
    struct BucketRec *rec;  // [rows] sample records, in bucket order
    int *bcnt;          // [nbuckets] samples per bucket (count pass)
    int *bstart;        // [nbuckets + 1] first row of each bucket (exclusive scan of bcnt)
    int *bcur;          // [nbuckets] next free row of each bucket (place pass)
    int *sidx;          // [B][G*KK][N] bucket row of each sample; -1 no corner inside
    int ntx, nty;       // cell tiles per row / column
    float *ring;        // [nbuckets][kRing][Cgp] grad_input sums of each window's border ring
    // grad_input written directly by the per-cell kernel and ring_final_kernel
    // (no fp32 accumulator): the caller's buffer, whether it is channels-last
    // [B][H][W][C] (else [B][C][H][W]), and whether 8-element runs take vector
    // stores there (NCHW: W % 8 == 0; channels-last: C and C/G multiples of
    // 8; both with a 16-byte aligned base)
    void *gi_out;
    int gi_nhwc, gi_vec;
    // offset / mask (and grad_offset / grad_mask) elements between images, and
    // whether the mask buffer holds logits (see mask_value; grad_mask is then
    // the gradient of the logits)
    long long off_bs, msk_bs;
    int msk_logit;
    // grad_weight work items: gw_nch chunks per M chunk.  Ungrouped (gw_cog
    // 0): every chunk.  Weight groups whose chunks never mix: an M chunk of
    // group w = m0 / gw_cog walks only that group's chunks tap*gw_cpt +
    // w*gw_cpw + i, i < gw_cpw (the other blocks of the block-diagonal packed
    // weight are zero and their grad_weight is not kept).
    int gw_nch, gw_cpt, gw_cpw, gw_cog;
};

// Eight consecutive elements as 16-byte stores (dst 16-byte aligned).
template <typename T> __device__ __forceinline__ void store8(T *dst, const T (&v)[8]) {
    if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<uint4 *>(dst) = __builtin_bit_cast(uint4, v);
    } else {
        uint4 *d = reinterpret_cast<uint4 *>(dst);
        d[0] = make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
        d[1] = make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7]));
    }
}

// Packed chunk index of the j-th grad_weight chunk of the M chunk at row m0.
__device__ __forceinline__ int gw_chunk(const BwdParams &p, int j, int m0) {
    if (p.gw_cog == 0) return j;
    const int tap = j / p.gw_cpw;
    return tap * p.gw_cpt + (m0 / p.gw_cog) * p.gw_cpw + (j - tap * p.gw_cpw);
}

// Element type of the masked column-gradient rows the column-gradient kernel
// hands to the grad_input gather: the call type, except bf16, whose 8-bit
// significand would add a rounding that the reference's fp32 col2im
// (com.cu:553-609) does not have.  bf16 rows are fp16 with one power-of-two
// scale per 32 channels (block floating point, kRowScaled): the largest
// magnitude of the 32 is brought to [2^14, 2^15) before the rounding to fp16,
// so every value keeps an 11-bit significand down to 2^-14 of its block's
// largest (subnormal below), and the block's exponent spans bf16's range.
// The scale codes live in BwdParams::rsc, one byte per 32 channels of a row.
template <typename T> struct RowOf { typedef T type; };
template <> struct RowOf<bf16> { typedef f16 type; };
template <typename T> constexpr bool kRowScaled = std::is_same<T, bf16>::value;
constexpr int row_elem_bytes(int dtype) { return dtype == DCN2_F32 ? 4 : 2; }
constexpr bool row_scaled(int dtype) { return dtype == DCN2_BF16; }

// Value of lane l ^ 1 / l ^ 2 (within each group of 4 lanes), by DPP quad permutes.
__device__ __forceinline__ float quad_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float quad_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
}

// Scale of one 32-channel block of a bf16 hand-off row, held by a quad of
// lanes with 8 values each (every lane of the quad calls this).  Returns the
// factor 2^s the values are multiplied by before the rounding to fp16, s =
// min(141 - e, 127) for the biased exponent e of the block's largest
// magnitude, and sets `code` = 127 - s, from which the consumers rebuild
// 2^-s (row_unscale; a block below 2^-113 gets code 0, read back as 0).
// NaN values stay NaN (fmaxf skips them) and infinities stay infinite.
__device__ __forceinline__ float row_block_scale(const float (&v)[8], unsigned &code) {
    float mx = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[e]));
    mx = fmaxf(mx, quad_xor1(mx));
    mx = fmaxf(mx, quad_xor2(mx));
    const int sc = min(141 - (int)(__float_as_uint(mx) >> 23), 127);
    code = (unsigned)(127 - sc);
    return __int_as_float((sc + 127) << 23);
}
__device__ __forceinline__ float row_unscale(unsigned code) { return __int_as_float(code << 23); }

// Buffer offset at or past one image's gO bytes (a load there reads 0); the
// kernels that read gO through it require Cout*N*sizeof(T) <= kGoOutOfRange.
constexpr int kGoOutOfRange = 0x7ffffff0;

// Cell tiles of the grad_input gather: a sample with floor corner (y0, x0)
// belongs to cell (y0+1, x0+1) of the (H+1) x (W+1) cell grid, and cells are
// grouped in kCellTile x kCellTile tiles, one bucket per (image, group, tile).
constexpr int kCellTile = 16;
// The pixels a tile's cells reach form a (kCellTile+1)^2 window whose border
// ring (kRing pixels) it shares with the neighbouring tiles.
constexpr int kRing = 4 * kCellTile;
static_assert(kRing == kGatherRing, "workspace sizing uses kGatherRing");

// Position of window pixel (py, px) in its border ring: the top row, the
// bottom row, then the left and right columns without their corners.
__device__ __forceinline__ int ring_index(int py, int px) {
    constexpr int TS = kCellTile, TW = kCellTile + 1;
    return py == 0 ? px : py == TS ? TW + px : px == 0 ? 2 * TW + py - 1 : 2 * TW + TS - 1 + py - 1;
}

// Per-pixel sampling record written by the reduction phase for the
// grad_input phase.  mode 0: no corner inside the image (nothing to add);
// 1: placed in its cell-tile bucket (write the masked column-gradient row).
struct Desc {
    int off[4];
    float w[4];  // masked bilinear weight of each corner, 0 outside the image
    int sidx;    // bucket row of the masked column gradient
    int mode;
    int pad0, pad1;
    // the last 16 bytes (DescFrac) are what the corner-sum reduction reads
    float m;     // mask value
    int valid;   // bit q: corner q inside the image
    float ly, lx;  // bilinear fractions
};
struct DescFrac {
    float m;
    int valid;
    float ly, lx;
};
static_assert(sizeof(Desc) == 64 && offsetof(Desc, m) % 16 == 0, "Desc is four 16-byte pieces");

// Claims one entry of counter `key` for this lane when `want`;
// wavefront-aggregated: one atomic per distinct key among the wave's lanes.
// Returns the counter's value before this lane's claim, or -1 when !want.
__device__ __forceinline__ int bucket_append(bool want, int key, int *ctr) {
    const int lane = threadIdx.x & 63;
    unsigned long long active = __ballot(want);
    int slot = -1;
    while (active) {
        const int leader = __ffsll((long long)active) - 1;
        const int lkey = __shfl(key, leader, 64);
        const unsigned long long same = __ballot(want && key == lkey) & active;
        int base = 0;
        if (lane == leader) base = atomicAdd(ctr + lkey, __popcll(same));
        base = __shfl(base, leader, 64);
        if ((same >> lane) & 1ull) slot = base + __popcll(same & ((1ull << lane) - 1ull));
        active &= ~same;
    }
    return slot;
}

template <typename T, int KPL> struct FragSet;
template <typename T> struct FragSet<T, 1> {
    template <typename F> static __device__ __forceinline__ void set(F &f, int, T v) { f = v; }
};
template <typename T> struct FragSet<T, 8> {
    template <typename F> static __device__ __forceinline__ void set(F &f, int e, T v) { f[e] = v; }
};

// f(integral_constant<int, I>) for I = B .. E-1, unrolled at compile time
// (for builtins whose operand must be a constant).
template <int B, int E, typename F> __device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
    return __shfl_xor(v, mask, 64);
}

// ---------------------------------------------------------------------------
// Bucket pre-passes of the grad_input hand-off.  Every sample (image, offset
// plane g*KK + tap, output pixel) with a corner inside the image belongs to
// the bucket of its cell tile.  Three launches place the samples in exactly
// sized buckets:
//   count  samples per bucket -> bcnt;
//   scan   bstart = exclusive prefix sum of bcnt (and bcur = bstart);
//   place  each sample claims a row of its bucket from bcur, writes its
//          record there and its row to sidx (-1: no corner inside),
// so the column-gradient kernel only reads one int per sample, and the
// buckets hold any distribution of samples (a learned offset field that pulls
// every sample into one tile included) in at most B*G*KK*N rows.  Count and
// place compute the sample position exactly as the column-gradient kernel
// does, so both passes see the same buckets.
//
// A workgroup takes kBucketSPT*256 consecutive pixels of one offset plane and
// counts its samples per cell tile in LDS (the LDS atomic's return value is
// the sample's rank inside the workgroup); then one global atomic per
// (workgroup, cell tile) adds its count (count pass) or claims a range of the
// bucket's rows (place pass).  Claiming rows with one global atomic per wave
// instead serialises thousands of atomics on each bucket counter.
//
// With at most kBucketFold buckets in all the place pass also does the scan:
// each workgroup sums the counts of the buckets before its image and group
// and scans those of its own tiles (a few thousand L2-resident ints), claims
// rows relative to the bucket start (bcur then starts at 0), and the first
// workgroup of each (image, group) writes its bucket starts for the later
// kernels.  That saves the one-workgroup scan launch between the passes.
constexpr int kBucketTab = 8191;   // cell tiles of one image the LDS tables may hold (2 * 8191 + 1 ints: 64 KB)
constexpr int kBucketSPT = 4;      // samples per thread
constexpr int kBucketFold = 4096;  // buckets up to which the place pass scans the counts itself

struct BucketSample {
    SamplePos sp;
    bool any;
    int tkey;  // cell tile inside the image: (cy / kCellTile) * ntx + cx / kCellTile
};

__device__ __forceinline__ BucketSample bucket_sample(const BwdParams &p, const void *offset_v,
                                                      int esz_is_f32, int is_bf16, int b,
                                                      int plane, int n) {
    const int N = p.Ho * p.Wo, KK = p.kh * p.kw;
    const int tap = plane % KK;
    const int ki = tap / p.kw, kj = tap - ki * p.kw;
    const bool live = n < N;
    const int nn = live ? n : 0;
    const int oy = nn / p.Wo, ox = nn - oy * p.Wo;
    const size_t ob = (size_t)b * p.off_bs + (size_t)plane * 2 * N + nn;
    float dy, dx;
    if (esz_is_f32) {
        dy = ((const float *)offset_v)[ob];
        dx = ((const float *)offset_v)[ob + N];
    } else if (is_bf16) {
        dy = to_f32(((const bf16 *)offset_v)[ob]);
        dx = to_f32(((const bf16 *)offset_v)[ob + N]);
    } else {
        dy = to_f32(((const f16 *)offset_v)[ob]);
        dx = to_f32(((const f16 *)offset_v)[ob + N]);
    }
    const float y = (float)(oy * p.sh - p.ph + ki * p.dh) + dy;
    const float x = (float)(ox * p.sw - p.pw + kj * p.dw) + dx;
    BucketSample r;
    r.sp = sample_pos(y, x, p.H, p.W);
    r.any = live && (r.sp.vy0 || r.sp.vy1) && (r.sp.vx0 || r.sp.vx1);
    r.tkey = ((r.sp.y0 + 1) / kCellTile) * p.ntx + (r.sp.x0 + 1) / kCellTile;
    return r;
}

// Places a sample's record (BucketRec).  Row `row` of the bucket storage is
// written only if it lies inside the bucket's range, so the storage is never
// written out of bounds, whatever the counts.
__device__ __forceinline__ int place_sample(const BwdParams &p, const BucketSample &bs, int key,
                                            int row) {
    if (row < 0 || row >= p.bstart[key + 1]) return -1;
    p.rec[row] = BucketRec{(bs.sp.y0 & 0xffff) | (int)((unsigned)bs.sp.x0 << 16), bs.sp.ly, bs.sp.lx};
    return row;
}

// PLACE = false: the count pass (bcnt); true: the place pass (bcur, rec, sidx).
template <bool PLACE>
__global__ __launch_bounds__(256) void dcn2_bucket_kernel(const BwdParams p, const void *offset_v,
                                                          int esz_is_f32, int is_bf16, int fold) {
    // [nty * ntx] per-tile counts, then (place pass) first rows; the place
    // pass also keeps the tiles' bucket starts, [nty * ntx + 1].  Sized at
    // launch, so small images run many workgroups per CU.
    extern __shared__ int tab[];
    __shared__ int wsum[4];
    const int N = p.Ho * p.Wo, KK = p.kh * p.kw;
    const int tid = threadIdx.x, ntile = p.nty * p.ntx;
    int *const tst = tab + ntile;  // (place pass only)
    const int plane = blockIdx.y, b = blockIdx.z, g = plane / KK;
    const int key0 = (b * p.G + g) * ntile;
    const int n_base = blockIdx.x * 256 * kBucketSPT;
    for (int i = tid; i < ntile; i += 256) tab[i] = 0;
    // Folded scan (place pass): tst[i] = bcnt[0] + ... + bcnt[key0 + i - 1],
    // i = 0..ntile (every count is complete: the count pass has ended).
    // Thread t holds counts 16t .. 16t + 15 from four independent 16-byte
    // loads, issued before the samples' offset loads so that both are in
    // flight together, through a buffer over the first key0 + ntile counts
    // rounded up to whole 16-byte pieces (bcnt has room for them; pieces past
    // it read 0); counts past key0 + ntile are set to 0.
    static_assert(kBucketFold == 256 * 16, "16 counts per thread");
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const int nb = key0 + ntile, lane = tid & 63;
    int v[16];
    if (PLACE && fold) {
        const __amdgpu_buffer_rsrc_t crs =
            __builtin_amdgcn_make_buffer_rsrc(p.bcnt, (short)0, ((nb + 3) & ~3) * (int)sizeof(int), 0x00020000);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 r = __builtin_amdgcn_raw_buffer_load_b128(crs, (tid * 16 + 4 * q) * 4, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * q + e] = (int)r[e];
        }
    }
    __syncthreads();
    int rank[kBucketSPT];
    BucketSample bsk[kBucketSPT];  // the place pass keeps the positions (no second computation)
#pragma unroll
    for (int k = 0; k < kBucketSPT; ++k) {
        const BucketSample bs =
            bucket_sample(p, offset_v, esz_is_f32, is_bf16, b, plane, n_base + k * 256 + tid);
        rank[k] = bs.any ? atomicAdd(tab + bs.tkey, 1) : -1;
        if constexpr (PLACE) bsk[k] = bs;
    }
    int sum = 0, incl = 0;
    if (PLACE && fold) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            v[e] = tid * 16 + e < nb ? v[e] : 0;
            sum += v[e];
        }
        incl = sum;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int o = __shfl_up(incl, d, 64);
            if (lane >= d) incl += o;
        }
        if (lane == 63) wsum[tid >> 6] = incl;
    }
    __syncthreads();
    if (PLACE && fold) {
        int run = incl - sum;
        for (int w = 0; w < (tid >> 6); ++w) run += wsum[w];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int j = tid * 16 + e;
            if (j >= key0 && j < nb) tst[j - key0] = run;
            run += v[e];
        }
        if (tid == 255) tst[ntile] = run;  // (the counts past nb are 0): the total
    } else if (PLACE) {
        for (int i = tid; i <= ntile; i += 256) tst[i] = p.bstart[key0 + i];
    }
    if constexpr (PLACE) __syncthreads();
    if (PLACE && fold && blockIdx.x == 0 && plane % KK == 0)
        for (int i = tid; i <= ntile; i += 256) p.bstart[key0 + i] = tst[i];
    int *ctr = (PLACE ? p.bcur : p.bcnt) + (size_t)key0;
    for (int i = tid; i < ntile; i += 256) {
        const int c = tab[i];
        // first row of this workgroup's range (bcur counts from the bucket
        // start when folded, holds absolute rows otherwise)
        if (c) tab[i] = (PLACE && fold ? tst[i] : 0) + atomicAdd(ctr + i, c);
    }
    if constexpr (PLACE) {
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kBucketSPT; ++k) {
            const int n = n_base + k * 256 + tid;
            if (n >= N) continue;
            int sx = -1;
            if (rank[k] >= 0) {
                // Row of the sample; written only inside the bucket's range, so
                // the storage is never written out of bounds, whatever the counts.
                const BucketSample &bs = bsk[k];
                const int row = tab[bs.tkey] + rank[k];
                if (row >= 0 && row < tst[bs.tkey + 1]) {
                    p.rec[row] = BucketRec{(bs.sp.y0 & 0xffff) | (int)((unsigned)bs.sp.x0 << 16), bs.sp.ly,
                                           bs.sp.lx};
                    sx = row;
                }
            }
            p.sidx[((size_t)b * p.G * KK + plane) * N + n] = sx;
        }
    }
}

// The same with one global atomic per (wave, bucket), for images with more
// cell tiles than kBucketTab.
template <bool PLACE>
__global__ __launch_bounds__(256) void dcn2_bucket_global_kernel(const BwdParams p,
                                                                 const void *offset_v,
                                                                 int esz_is_f32, int is_bf16) {
    const int N = p.Ho * p.Wo, KK = p.kh * p.kw;
    const int n = blockIdx.x * 256 + threadIdx.x;
    const int plane = blockIdx.y, b = blockIdx.z, g = plane / KK;
    const BucketSample bs = bucket_sample(p, offset_v, esz_is_f32, is_bf16, b, plane, n);
    const int key = (b * p.G + g) * p.nty * p.ntx + bs.tkey;
    const int row = bucket_append(bs.any, key, PLACE ? p.bcur : p.bcnt);
    if constexpr (PLACE) {
        const int sx = bs.any ? place_sample(p, bs, key, row) : -1;
        if (n < N) p.sidx[((size_t)b * p.G * KK + plane) * N + n] = sx;
    }
}

// bstart[i] = bcnt[0] + ... + bcnt[i-1] for i = 0..n, and bcur = bstart:
// one workgroup; thread t scans a contiguous run of ceil(n / 1024) counts.
__global__ __launch_bounds__(1024) void dcn2_bucket_scan_kernel(const int *__restrict__ bcnt,
                                                                int *__restrict__ bstart,
                                                                int *__restrict__ bcur, int n) {
    __shared__ int wsum[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int per = (n + 1023) / 1024;
    const int i0 = min(tid * per, n), i1 = min(i0 + per, n);
    int s = 0;
    for (int i = i0; i < i1; ++i) s += bcnt[i];
    int incl = s;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int run = incl - s;
    for (int w = 0; w < wave; ++w) run += wsum[w];
    for (int i = i0; i < i1; ++i) {
        bstart[i] = run;
        bcur[i] = run;
        run += bcnt[i];
    }
    if (tid == 1023) bstart[n] = run;  // thread 1023's run ends at n: the total
}

// Sink of the stores the column-gradient kernel issues with nothing to store
// (its contents are never read; each device holds its own copy).  Waves of
// different workgroups use different 2 KiB pieces, so that such stores do
// not all queue on one cache line.
constexpr int kTrashBytes = 64 * 1024;
__device__ __attribute__((aligned(16))) unsigned char dcn2_trash[kTrashBytes];

// ---------------------------------------------------------------------------
// Column-gradient kernel: grad_offset, grad_mask and grad_input.
// 512 threads; BN = 128 output pixels of one image per block.
// ALDS: the W'^T fragments of a chunk (Mp*128 bytes, Mp <= 256) are staged in
// LDS two chunks ahead; otherwise every wave reads its fragments from memory.
//
// The K chunks run as a software pipeline with one barrier per step.  Step c:
//   reduces chunk c (gathered and multiplied one step earlier) to
//   grad_offset / grad_mask,
//   loads W'^T and the offsets of chunk c+2,
//   issues the corner gathers of chunk c+1 and stores its descriptors,
//   computes the column gradient of chunk c+1 on the matrix cores,
//   hands chunk c's column gradient to grad_input,
// so a gather lands while the next MFMA and hand-off run, and the
// vector-memory traffic of one chunk overlaps the matrix work of the next
// instead of alternating with it.  The column-gradient stage and the
// descriptors are double-buffered by chunk parity.  The stores of a step do
// not depend on the data (a row with nothing to store goes to dcn2_trash),
// so the compiler's in-order count of outstanding memory operations stays
// exact and a gather is waited for without waiting for later stores.
template <typename T, int MCH, bool ALDS, bool ONEM>
__global__ __launch_bounds__(512) void dcn2_colgrad_kernel(const BwdParams p) {
    using M = Mma<T>;
    using frag = typename M::frag;
    constexpr int KC = M::KC, KPL = M::KPL, KSTEP = M::KSTEP;
    constexpr int BN = 128;
    constexpr int NB = (KC / 32) * (BN / 32);  // 32x32 blocks of one chunk (8 or 4)
    constexpr int WPB = 8 / NB;                // waves sharing one block's M reduction
    constexpr int MPW = MCH / WPB;             // M range of one wave per M chunk
    constexpr int NMS = MPW / KSTEP;           // MFMA steps per wave per M chunk
    constexpr int LDC = KC + 4;                // pitch (floats) of the column gradient
    constexpr int QPP = 512 / BN;              // lanes per pixel in the reduction phase
    constexpr int CPL = KC / QPP;              // channels per lane there
    constexpr int E = Unpack<T>::E;
    static_assert(CPL * sizeof(T) == 32, "reduction lane covers 32 bytes per corner");

    // LDS, carved from one array so that nothing is padded:
    //   sCG[2][WPB][BN][LDC] floats  column gradient of a chunk pair
    //   sD[2][BN]                    descriptors of a chunk pair
    //   sA[2][kAVec] uint4           staged W'^T of two chunks (ALDS only)
    constexpr int kAVec = 2048;  // 16-byte vectors of one staged chunk (Mp = 256)
    constexpr size_t kCGBytes = sizeof(float) * WPB * BN * LDC;
    constexpr size_t kDBytes = sizeof(Desc) * BN;
    constexpr size_t kABytes = ALDS ? sizeof(uint4) * kAVec : 0;
    static_assert(kCGBytes % 16 == 0 && kDBytes % 16 == 0, "16-byte aligned carving");
    __shared__ __attribute__((aligned(16))) char smem[2 * (kCGBytes + kDBytes + kABytes)];
    typedef float CGStage[WPB][BN][LDC];
    CGStage *const sCG = reinterpret_cast<CGStage *>(smem);
    Desc(*const sD)[BN] = reinterpret_cast<Desc(*)[BN]>(smem + 2 * kCGBytes);
    uint4(*const sA)[kAVec] = reinterpret_cast<uint4(*)[kAVec]>(smem + 2 * (kCGBytes + kDBytes));

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int blk = wave % NB, wr = wave / NB;
    const int kb = blk / (BN / 32), nb = blk - kb * (BN / 32);
    // tiles handed to the XCDs in contiguous ranges (xcd_remap): an XCD's
    // blocks work on neighbouring pixel rows, so the corner lines their
    // samples share are fetched into its L2 once
    const int tile = xcd_remap((int)(blockIdx.y * gridDim.x + blockIdx.x), (int)(gridDim.x * gridDim.y));
    const int b = tile / (int)gridDim.x, n0 = (tile - b * (int)gridDim.x) * BN;
    const int N = p.Ho * p.Wo, KK = p.kh * p.kw, cs = p.G * p.Cgp;
    const int cpg = p.Cgp / KC, nch = KK * p.G * cpg, nmc = p.Mp / MCH;

    const T *__restrict__ xt = (const T *)p.xt + (size_t)b * p.H * p.W * cs;
    const T *__restrict__ offs = (const T *)p.offset + (size_t)b * p.off_bs;
    const T *__restrict__ msk = p.mask ? (const T *)p.mask + (size_t)b * p.msk_bs : nullptr;
    const T *__restrict__ go = (const T *)p.gout + (size_t)b * p.Cout * N;
    const T *__restrict__ wt = (const T *)p.wt;
    T *__restrict__ goff = (T *)p.goff + (size_t)b * p.off_bs;
    T *__restrict__ gmask = p.gmask ? (T *)p.gmask + (size_t)b * p.msk_bs : nullptr;

    // gO fragments (MFMA B operand, [m][n]): n = this wave's 32-pixel block.
    frag gfr[NMS];
    // (channels-last gO: a fragment's KPL rows of one pixel are contiguous,
    // one 16-byte load for 2-byte types when Cout % 8 == 0)
    auto load_go = [&](int mc) __attribute__((always_inline)) {
        const int n = n0 + nb * 32 + (lane & 31);
#pragma unroll
        for (int s = 0; s < NMS; ++s) {
            const int m0s = mc * MCH + wr * MPW + s * KSTEP + (lane >> 5) * KPL;
            if (p.go_nhwc) {
                const T *gp = go + (size_t)n * p.Cout + m0s;
                if (KPL == 8 && p.go_vec && n < N && m0s < p.Cout) {
                    gfr[s] = *reinterpret_cast<const frag *>(gp);
                } else {
#pragma unroll
                    for (int e = 0; e < KPL; ++e)
                        FragSet<T, KPL>::set(gfr[s], e,
                                             (n < N && m0s + e < p.Cout) ? gp[e] : (T)0.0f);
                }
            } else {
#pragma unroll
                for (int e = 0; e < KPL; ++e) {
                    const int m = m0s + e;
                    const T v = (n < N && m < p.Cout) ? go[(size_t)m * N + n] : (T)0.0f;
                    FragSet<T, KPL>::set(gfr[s], e, v);
                }
            }
        }
    };
    // The same fragments for 2-byte types with 16-byte gO rows (one M chunk):
    // the block's gO tile [MCH][BN] is read with 16-byte buffer loads, 16
    // consecutive lanes per row (the element loads above cost one instruction
    // per value), issued before the sampling of chunk 0 and stored into the
    // column-gradient area of the LDS after it; then every fragment is two
    // transposing LDS reads (ds_read_b64_tr_b16: within 16 lanes, lane i
    // receives element i%4 of the 4-element pieces that lanes i/4, 4 + i/4,
    // 8 + i/4 and 12 + i/4 point at).  Lane L of a 16-lane group points at 4
    // consecutive pixels of row L/4 of the fragment's 4-row half, so lane i
    // receives rows 0..3 of that half at pixel i.  Row m keeps its 32-byte
    // blocks XOR-permuted by m%4, which puts the 4 rows of one read on
    // distinct banks.  Rows past Cout and pixels past N read 0 (buffer range).
    constexpr int GQ = (sizeof(T) == 2 ? MCH * (BN / 8) : 512) / 512;  // 16-byte pieces per thread
    const bool go_stage = ONEM && sizeof(T) == 2 && p.go_vec && !p.go_nhwc &&
                          (size_t)p.Cout * N * sizeof(T) <= (size_t)kGoOutOfRange;
    uint4 gst[GQ];
    auto go_stage_issue = [&]() __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<T *>(go), (short)0, (int)((size_t)p.Cout * N * sizeof(T)), 0x00020000);
#pragma unroll
        for (int q = 0; q < GQ; ++q) {
            const int idx = tid + 512 * q, m = idx / (BN / 8), n = n0 + (idx % (BN / 8)) * 8;
            const int off = (int)(((unsigned)m * (unsigned)N + (unsigned)n) * sizeof(T));
            gst[q] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                   rs, n < N ? off : kGoOutOfRange, 0, 0));
        }
    };
    T *const gstg = reinterpret_cast<T *>(smem);  // [MCH][BN], inside the sCG area
    static_assert(sizeof(T) * MCH * BN <= kCGBytes * 2, "gO stage fits the column-gradient area");
    auto go_stage_store = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < GQ; ++q) {
            const int idx = tid + 512 * q, m = idx / (BN / 8), n = (idx % (BN / 8)) * 8;
            *reinterpret_cast<uint4 *>(gstg + m * BN + (n ^ ((m & 3) << 4))) = gst[q];
        }
    };
    auto go_stage_read = [&]() __attribute__((always_inline)) {
        if constexpr (sizeof(T) == 2) {
            typedef short s16x4 __attribute__((ext_vector_type(4)));
            const int g = lane >> 4, li = lane & 15;
#pragma unroll
            for (int s = 0; s < NMS; ++s) {
                s16x4 h[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int m = wr * MPW + s * KSTEP + 8 * (g >> 1) + 4 * hh + (li >> 2);
                    const int nl = nb * 32 + 16 * (g & 1) + 4 * (li & 3);
                    h[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) s16x4 *)(gstg + m * BN +
                                                                    (nl ^ ((m & 3) << 4))));
                }
                gfr[s] = __builtin_bit_cast(frag, __builtin_shufflevector(h[0], h[1], 0, 1, 2, 3, 4, 5,
                                                                           6, 7));
            }
        }
    };

    // Reduction-phase identity: pixel pr, channel quarter lq.
    const int pr = tid / QPP, lq = tid - pr * QPP;
    const int nr = n0 + pr;
    const bool live = nr < N;
    int oyr = 0, oxr = 0;
    if (live) {
        oyr = nr / p.Wo;
        oxr = nr - oyr * p.Wo;
    }
    float racc[3] = {0.0f, 0.0f, 0.0f};  // grad_mask, grad_off_y, grad_off_x of (pr, tap, g)
    int gmode = 0, gsidx = 0;             // grad_input mode of (pr, tap, g), see Desc
    const int *__restrict__ sidx = p.sidx + (size_t)b * p.G * KK * N;

    // W'^T staging: chunk c's fragments are Mp*8 consecutive 16-byte vectors
    // (pack_weight_kernel layout 1 is k-block major); each thread moves four
    // of them, loaded at the start of step c-2 and written to the LDS buffer
    // of chunk c's parity at its end.  Vectors past Mp*8 (Mp < 256) re-read
    // the last one and land in the unused tail of the buffer, so neither the
    // loads nor the writes sit in a branch (the compiler would otherwise fuse
    // each load with its write and wait for it on the spot).
    const int avec = p.Mp * 8;
    const uint4 *__restrict__ wtv = (const uint4 *)p.wt;
    uint4 apf0, apf1, apf2, apf3;  // (named registers: as an array it was put in scratch)
    auto a_prefetch = [&](int c) __attribute__((always_inline)) {
        if constexpr (ALDS) {
            const uint4 *src = wtv + (size_t)c * avec;
            apf0 = src[min(tid, avec - 1)];
            apf1 = src[min(tid + 512, avec - 1)];
            apf2 = src[min(tid + 1024, avec - 1)];
            apf3 = src[min(tid + 1536, avec - 1)];
        }
    };
    auto a_commit = [&](int buf) __attribute__((always_inline)) {
        if constexpr (ALDS) {
            sA[buf][tid] = apf0;
            sA[buf][tid + 512] = apf1;
            sA[buf][tid + 1024] = apf2;
            sA[buf][tid + 1536] = apf3;
        }
    };

    // Chunk c = (tap*G + g)*cpg + cc, tap = ki*kw + kj.  The steps walk the
    // chunks in order, so the ids are advanced with compares instead of being
    // divided out of c (runtime divisors expand to long scalar sequences, and
    // the scalar unit is shared by the CU's waves).
    struct ChunkId {
        int cc, g, tap, ki, kj;
    };
    auto chunk_next = [&](ChunkId r) __attribute__((always_inline)) {
        if (++r.cc == cpg) {
            r.cc = 0;
            if (++r.g == p.G) {
                r.g = 0;
                ++r.tap;
                if (++r.kj == p.kw) {
                    r.kj = 0;
                    ++r.ki;
                }
            }
        }
        return r;
    };

    // Offsets, mask and bucket row of (pr, chunk), loaded two steps ahead.
    struct OM {
        T dy, dx, m;
        int sx;
    };
    auto load_om = [&](const ChunkId &id, OM &o) __attribute__((always_inline)) {
        const int plane = id.g * KK + id.tap;
        const int nn = live ? nr : 0;
        const size_t ob = (size_t)plane * 2 * N + nn;
        o.dy = offs[ob];
        o.dx = offs[ob + N];
        o.m = msk ? msk[(size_t)plane * N + nn] : (T)1.0f;
        o.sx = sidx[(size_t)plane * N + nn];
    };
    // This thread's corner gathers of the chunk sampled last.
    uint4 raw[4][2];
    // this lane's 32 bytes of dcn2_trash (a wave uses one 2 KiB piece)
    uint4 *const trash_v = reinterpret_cast<uint4 *>(dcn2_trash) +
                           ((blockIdx.x * 8 + wave) % (kTrashBytes / 2048)) * 128 + lane * 2;
    T *const trash_t = reinterpret_cast<T *>(trash_v);

    // Sampling of chunk c (offsets o): corner gathers, and the descriptor of
    // pixel pr into sD[X].
    auto sample = [&](int X, const ChunkId &id, const OM &o) __attribute__((always_inline)) {
        const int ki = id.ki, kj = id.kj;
        SamplePos sp;
        float mv = 0.0f;
        if (live) {
            const float y = (float)(oyr * p.sh - p.ph + ki * p.dh) + to_f32(o.dy);
            const float x = (float)(oxr * p.sw - p.pw + kj * p.dw) + to_f32(o.dx);
            mv = mask_value(to_f32(o.m), p.msk_logit);
            sp = sample_pos(y, x, p.H, p.W);
        } else {
            sp = sample_pos(-2.0f, -2.0f, p.H, p.W);
        }
        const Corners cr = make_corners(sp, mv, p.W, cs);
        const int cbase = id.g * p.Cgp + id.cc * KC + lq * CPL;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint4 *src = reinterpret_cast<const uint4 *>(xt + cr.off[q] + cbase);
            raw[q][0] = src[0];
            raw[q][1] = src[1];
        }
        if (id.cc == 0) {
            gmode = o.sx >= 0 ? 1 : 0;
            gsidx = o.sx;
        }
        if (lq == 0) {
            Desc d;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                d.off[q] = cr.off[q];
                d.w[q] = cr.w[q];
            }
            d.sidx = gsidx;
            d.mode = gmode;
            d.pad0 = d.pad1 = 0;
            d.m = mv;
            d.valid = (sp.vy0 && sp.vx0 ? 1 : 0) | (sp.vy0 && sp.vx1 ? 2 : 0) |
                      (sp.vy1 && sp.vx0 ? 4 : 0) | (sp.vy1 && sp.vx1 ? 8 : 0);
            d.ly = sp.ly;
            d.lx = sp.lx;
            sD[X][pr] = d;
        }
    };

    // Column gradient of chunk c (block (kb, nb), M share wr) into sCG[X].
    auto colgrad = [&](int X, int c) __attribute__((always_inline)) {
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
        // A = W'^T in fragment order (pack_weight_kernel layout 1): the
        // fragment (row block c*KC/32 + kb, step ms) is one contiguous run.
        const T *wrow = wt + ((size_t)(c * KC / 32 + kb) * (p.Mp / KSTEP) + wr * (MPW / KSTEP)) *
                                 64 * KPL + lane * KPL;
        const T *arow = reinterpret_cast<const T *>(&sA[X][0]) +
                        ((size_t)kb * (p.Mp / KSTEP) + wr * (MPW / KSTEP)) * 64 * KPL + lane * KPL;
        if constexpr (ONEM) {
            // gO is resident: no memory access here, so the MFMAs never wait
            // for the gathers issued just before them
#pragma unroll
            for (int s = 0; s < NMS; ++s) {
                const frag a = *reinterpret_cast<const frag *>((ALDS ? arow : wrow) +
                                                               (size_t)s * 64 * KPL);
                acc = M::mma(a, gfr[s], acc);
            }
        } else {
            for (int mc = 0; mc < nmc; ++mc) {
                load_go(mc);
#pragma unroll
                for (int s = 0; s < NMS; ++s) {
                    const size_t fo = (size_t)(mc * (MCH / KSTEP) + s) * 64 * KPL;
                    const frag a = *reinterpret_cast<const frag *>((ALDS ? arow : wrow) + fo);
                    acc = M::mma(a, gfr[s], acc);
                }
            }
        }
        const int nl = nb * 32 + (lane & 31);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int kl = kb * 32 + 8 * j + 4 * (lane >> 5);
            *reinterpret_cast<f32x4 *>(&sCG[X][wr][nl][kl]) =
                f32x4{acc[4 * j], acc[4 * j + 1], acc[4 * j + 2], acc[4 * j + 3]};
        }
    };

    // Chunk c (parity X): grad_mask / grad_offset from corner sums over this
    // lane's channels.  The shuffles leave the sums in all QPP lanes of the
    // pixel, which all store the same values at the last chunk of its (tap,
    // group) (the lanes of a dead pixel store to dcn2_trash).
    auto reduce_corners = [&](int X, const ChunkId &id) __attribute__((always_inline)) {
        float cgv[CPL];
#pragma unroll
        for (int c4 = 0; c4 < CPL / 4; ++c4) {
            f32x4 v = *reinterpret_cast<const f32x4 *>(&sCG[X][0][pr][lq * CPL + 4 * c4]);
#pragma unroll
            for (int w2 = 1; w2 < WPB; ++w2)
                v += *reinterpret_cast<const f32x4 *>(&sCG[X][w2][pr][lq * CPL + 4 * c4]);
            cgv[4 * c4] = v[0];
            cgv[4 * c4 + 1] = v[1];
            cgv[4 * c4 + 2] = v[2];
            cgv[4 * c4 + 3] = v[3];
        }
        float S[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float s = 0.0f;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                float v[E];
                Unpack<T>::run(raw[q][u], v);
#pragma unroll
                for (int e = 0; e < E; ++e) s = fmaf(cgv[u * E + e], v[e], s);
            }
            S[q] = s;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma unroll
            for (int x = 1; x < QPP; x <<= 1) S[q] += shfl_xor_f(S[q], x);
        }
        // mask value, corner validity and fractions of the sample (one LDS read)
        const DescFrac f = *reinterpret_cast<const DescFrac *>(&sD[X][pr].m);
        const int vq = f.valid;
        const float S0 = (vq & 1) ? S[0] : 0.0f, S1 = (vq & 2) ? S[1] : 0.0f;
        const float S2 = (vq & 4) ? S[2] : 0.0f, S3 = (vq & 8) ? S[3] : 0.0f;
        const float ly = f.ly, lx = f.lx, hy = 1.0f - ly, hx = 1.0f - lx;
        const float mv = f.m;
        racc[0] += hy * hx * S0 + hy * lx * S1 + ly * hx * S2 + ly * lx * S3;
        racc[1] += mv * (hx * (S2 - S0) + lx * (S3 - S1));
        racc[2] += mv * (hy * (S1 - S0) + ly * (S3 - S2));
        if (id.cc == cpg - 1) {
            const size_t plane = (size_t)id.g * KK + id.tap;
            *(live ? goff + plane * 2 * N + nr : trash_t) = from_f32<T>(racc[1]);
            *(live ? goff + plane * 2 * N + N + nr : trash_t + 1) = from_f32<T>(racc[2]);
            // d/d(logit) of sigmoid = s (1 - s), s = the mask value used
            const float gm = p.msk_logit ? racc[0] * mv * (1.0f - mv) : racc[0];
            if (gmask) *(live ? gmask + plane * N + nr : trash_t + 2) = from_f32<T>(gm);
            racc[0] = racc[1] = racc[2] = 0.0f;
        }
    };

    // grad_input hand-off of chunk c (parity X): 8 lanes per pixel, 16 bytes
    // (EPL channels) per lane.  A bucketed sample stores its masked
    // column-gradient row (8 rows of 16-byte pieces per wave instruction) for
    // the gather kernel; a sample with no corner inside stores to dcn2_trash.
    auto handoff = [&](int X, const ChunkId &id) __attribute__((always_inline)) {
        typedef typename RowOf<T>::type R;
        constexpr int EPL = 16 / sizeof(T), LPP = KC / EPL, PPI = 64 / LPP;
        constexpr int NST = EPL * sizeof(R) / 16;  // 16-byte stores per lane
        static_assert(LPP == 8, "8 lanes cover one chunk row");
        const int co = lane % LPP, r = lane / LPP;
#pragma unroll
        for (int it = 0; it < BN / (8 * PPI); ++it) {
            const int pl = (it * 8 + wave) * PPI + r;
            const bool in = n0 + pl < N;
            const Desc d = sD[X][pl];
            float v[EPL];
#pragma unroll
            for (int e4 = 0; e4 < EPL / 4; ++e4) {
                f32x4 x = *reinterpret_cast<const f32x4 *>(&sCG[X][0][pl][co * EPL + 4 * e4]);
#pragma unroll
                for (int w2 = 1; w2 < WPB; ++w2)
                    x += *reinterpret_cast<const f32x4 *>(&sCG[X][w2][pl][co * EPL + 4 * e4]);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[4 * e4 + e] = x[e];
            }
            float mv8[EPL];
#pragma unroll
            for (int e = 0; e < EPL; ++e) mv8[e] = v[e] * d.m;
            uint4 *row = reinterpret_cast<uint4 *>((R *)p.cgm + (size_t)d.sidx * p.Cgp + id.cc * KC +
                                                   co * EPL);
            uint4 *dst = in && d.mode == 1 ? row : trash_v;
            if constexpr (kRowScaled<T>) {
                // lanes co 0-3 / 4-7 (quads) hold the chunk row's two 32-channel blocks
                unsigned code;
                const float f = row_block_scale(mv8, code);
#pragma unroll
                for (int e = 0; e < EPL; ++e) mv8[e] *= f;
                unsigned char *sc = in && d.mode == 1 && (co & 3) == 0
                                        ? p.rsc + (size_t)d.sidx * (p.Cgp / 32) + id.cc * 2 + (co >> 2)
                                        : reinterpret_cast<unsigned char *>(trash_v) + 8;
                *sc = (unsigned char)code;
            }
#pragma unroll
            for (int i = 0; i < NST; ++i) dst[i] = pack16<R>(mv8 + i * (16 / sizeof(R)));
        }
    };

    // Prologue: chunk 0 sampled and multiplied, W'^T of chunk 1 staged,
    // offsets of chunk 1 loaded.
    OM om_c, om_n;  // offsets of the chunk sampled next, and of the one after
    // Loads past the last chunk re-read the last chunk (clamped index) rather
    // than sitting in a branch: with every memory operation of a step issued
    // unconditionally the compiler's load counting stays exact across steps.
    const int last = nch - 1;
    if constexpr (ONEM) {
        if (go_stage) go_stage_issue();
        else load_go(0);
    }
    // ids of chunks c, c+1 and min(c+2, last) of the step
    ChunkId id0 = {0, 0, 0, 0, 0};
    ChunkId id1 = last >= 1 ? chunk_next(id0) : id0;
    ChunkId id2 = last >= 2 ? chunk_next(id1) : id1;
    load_om(id0, om_c);
    a_prefetch(0);
    load_om(id1, om_n);
    sample(0, id0, om_c);
    if (go_stage) go_stage_store();
    a_commit(0);
    a_prefetch(min(1, last));
    __syncthreads();
    if (go_stage) {
        go_stage_read();
        __syncthreads();  // colgrad(0) writes the column-gradient area
    }
    colgrad(0, 0);
    a_commit(1);
    om_c = om_n;
    __syncthreads();

    for (int c = 0; c < last; ++c) {
        const int X = c & 1, Y = X ^ 1;
        reduce_corners(X, id0);
        a_prefetch(min(c + 2, last));
        load_om(id2, om_n);
        sample(Y, id1, om_c);
        colgrad(Y, c + 1);
        handoff(X, id0);
        a_commit(X);  // chunk c+2 has chunk c's parity, and MFMA(c) is done
        om_c = om_n;
        id0 = id1;
        id1 = id2;
        if (c + 3 <= last) id2 = chunk_next(id2);
        __syncthreads();
    }
    reduce_corners(last & 1, id0);
    handoff(last & 1, id0);
}

// ---------------------------------------------------------------------------
// grad_weight kernel.  Block = one K chunk (blockIdx.y) x 32*MB output
// channels (blockIdx.z) x a strided subset of the pixel tiles (blockIdx.x).
// D[m][k] = sum_n gO[m][n] * col[k][n]; A = gO straight from global memory
// (rows are pixel-contiguous), B = re-sampled columns in LDS.
// 2-byte types keep the LDS stage as [k][n] with the 16-byte blocks of each
// row XOR-swizzled by h(k) = ((k & 15) ^ (k >> 3)) & 15 so that both the
// sampler's 2-byte stores and the MFMA's 16-byte reads are bank-conflict free.
template <typename T> struct GwLayout;
template <> struct GwLayout<float> {
    static constexpr bool kMajor = false;
};
template <> struct GwLayout<f16> {
    static constexpr bool kMajor = true;
};
template <> struct GwLayout<bf16> {
    static constexpr bool kMajor = true;
};

__device__ __forceinline__ int gw_swz(int k) { return ((k & 15) ^ (k >> 3)) & 15; }

// This kernel serves fp32 and gO rows that 16-byte loads cannot read (N % 8
// != 0 or an unaligned base); 2-byte types with aligned rows take
// dcn2_gradw_line_kernel below.  gO is read with guarded loads.
template <typename T, int MB, bool MASK>
__global__ __launch_bounds__(512) void dcn2_gradw_kernel(const BwdParams p) {
    using M = Mma<T>;
    using frag = typename M::frag;
    constexpr int KC = M::KC, KPL = M::KPL, KSTEP = M::KSTEP;
    constexpr int BN = 128, NKS = BN / KSTEP;
    constexpr int KB = KC / 32;
    constexpr int NBLK = MB * KB;
    constexpr int BPW = NBLK >= 16 ? 2 : 1;  // blocks per wave
    constexpr bool KMAJ = GwLayout<T>::kMajor;
    constexpr int LDN = KMAJ ? BN : KC + 4;  // pitch of the LDS stage (elements)
    constexpr int ROWS = KMAJ ? KC : BN;
    constexpr int CPS = KC / 4;
    static_assert(!KMAJ || BN == 128, "swizzle assumes 16 blocks of 8 per row");

    __shared__ __attribute__((aligned(16))) T sC[2][ROWS][LDN];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int mblk, kblk0;
    bool active;
    if constexpr (BPW == 2) {
        mblk = wave;
        kblk0 = 0;
        active = true;
    } else {
        mblk = wave / KB;
        kblk0 = wave - mblk * KB;
        active = wave < NBLK;
    }
    // Work item = (pixel-tile range sp, K chunk ch, M chunk mc), handed to XCDs
    // in contiguous ranges with the range index slowest, so one XCD works on
    // consecutive pixel tiles (same images) for all chunks.
    const int nmc = p.Mp / (32 * MB);
    const int wi = xcd_remap(blockIdx.x, p.splits * p.gw_nch * nmc);
    const int mc = wi % nmc, j = (wi / nmc) % p.gw_nch, sp = wi / (nmc * p.gw_nch);
    const int ch = gw_chunk(p, j, mc * 32 * MB);
    const bool do_bias = p.gb_acc != nullptr && j == 0 && kblk0 == 0 && active;
    const int mrow = mc * 32 * MB + mblk * 32 + (lane & 31);
    const int N = p.Ho * p.Wo, KK = p.kh * p.kw, cs = p.G * p.Cgp;
    const int T_total = p.B * p.tiles_per_img;
    // contiguous range of pixel tiles [t_begin, t_end) of this work item
    const int t_begin = (int)((long)T_total * sp / p.splits);
    const int t_end = (int)((long)T_total * (sp + 1) / p.splits);

    SampleGeo sg;
    sg.H = p.H; sg.W = p.W; sg.kh = p.kh; sg.kw = p.kw; sg.sh = p.sh; sg.sw = p.sw;
    sg.ph = p.ph; sg.pw = p.pw; sg.dh = p.dh; sg.dw = p.dw; sg.G = p.G; sg.Cgp = p.Cgp;
    sg.Wo = p.Wo; sg.N = N; sg.cs = cs; sg.KK = KK; sg.msk_logit = p.msk_logit;
    const ChunkEnt cp = ((const ChunkEnt *)p.tab)[ch];
    // Two sampler register sets / offset-mask sets alternate between even and
    // odd tiles (loop unrolled by two): offset/mask loads run 3 tiles ahead of
    // the MFMA, corner gathers 2 ahead, the LDS store 1 ahead.
    Sampler<T, 1, MASK> smp[2];
    smp[0].init(tid);
    smp[1].init(tid);
    SlotOM<T, 1> om[2];

    auto load_om_tile = [&](int t, SlotOM<T, 1> &o) __attribute__((always_inline)) {
        const int b = t / p.tiles_per_img, n0 = (t - b * p.tiles_per_img) * BN;
        smp[0].load_om(n0, cp.x, sg, tid, (const T *)p.offset + (size_t)b * p.off_bs,
                       MASK ? (const T *)p.mask + (size_t)b * p.msk_bs : nullptr, o);
    };
    auto issue_tile = [&](auto set_c, int t, const SlotOM<T, 1> &o) __attribute__((always_inline)) {
        constexpr int set = decltype(set_c)::value;
        const int b = t / p.tiles_per_img;
        smp[set].issue(cp, sg, (const T *)p.xt + (size_t)b * p.H * p.W * cs, o);
    };
    auto store_stage = [&](auto set_c, int buf) __attribute__((always_inline)) {
        constexpr int set = decltype(set_c)::value;
        const int pl = tid >> 2;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            float v[16 / sizeof(T)];
            smp[set].blend(0, u, v);
            if constexpr (KMAJ) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int k = smp[set].q * CPS + u * 8 + e;
                    sC[buf][k][((pl >> 3) ^ gw_swz(k)) * 8 + (pl & 7)] = (T)v[e];
                }
            } else {
                *reinterpret_cast<uint4 *>(&sC[buf][pl][smp[set].q * CPS + u * 4]) = pack16<T>(v);
            }
        }
    };

    f32x16 acc[BPW];
#pragma unroll
    for (int i = 0; i < BPW; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
    float bsum = 0.0f;

    const bool aligned = p.go_vec != 0;
    auto load_a = [&](frag &a, int t, int ks) __attribute__((always_inline)) {
        const int b = t / p.tiles_per_img, n0 = (t - b * p.tiles_per_img) * BN;
        const int n = n0 + ks * KSTEP + (lane >> 5) * KPL;
        if (p.go_nhwc) {  // channels-last: the KPL pixels of a row are Cout apart
            const T *col = (const T *)p.gout + (size_t)b * p.Cout * N + mrow;
#pragma unroll
            for (int e = 0; e < KPL; ++e) {
                const T v = (mrow < p.Cout && n + e < N) ? col[(size_t)(n + e) * p.Cout] : (T)0.0f;
                FragSet<T, KPL>::set(a, e, v);
            }
            return;
        }
        const T *row = (const T *)p.gout + ((size_t)b * p.Cout + mrow) * N;
        if (mrow < p.Cout && aligned && n + KPL <= N && KPL == 8) {
            a = *reinterpret_cast<const frag *>(row + n);
        } else {
#pragma unroll
            for (int e = 0; e < KPL; ++e) {
                const T v = (mrow < p.Cout && n + e < N) ? row[n + e] : (T)0.0f;
                FragSet<T, KPL>::set(a, e, v);
            }
        }
    };
    // gO fragments of a whole tile are prefetched one step ahead for 2-byte
    // types (8 registers of 16 bytes), in the set of the tile's parity (the
    // loop is unrolled by two, so no register copies); fp32 (64 one-float
    // steps) loads at use.
    constexpr bool PREA = KPL == 8;
    frag a_set[2][PREA ? NKS : 1];
    auto load_a_tile = [&](frag (&a)[PREA ? NKS : 1], int t) __attribute__((always_inline)) {
        if constexpr (PREA) {
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) load_a(a[ks], t, ks);
        }
    };

    auto mfma_tile = [&](auto s_c, int t) __attribute__((always_inline)) {
        constexpr int buf = decltype(s_c)::value;
        if (!active) return;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            frag a;
            if constexpr (PREA) {
                a = a_set[buf][ks];
            } else {
                load_a(a, t, ks);
                if (do_bias) {
                    if constexpr (KPL == 1) {
                        bsum += to_f32(a);
                    } else {
#pragma unroll
                        for (int e = 0; e < KPL; ++e) bsum += to_f32(a[e]);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < BPW; ++i) {
                const int k = (kblk0 + i) * 32 + (lane & 31);
                frag bf;
                if constexpr (KMAJ) {
                    const int nblk = ks * 2 + (lane >> 5);
                    bf = *reinterpret_cast<const frag *>(&sC[buf][k][(nblk ^ gw_swz(k)) * 8]);
                } else {
                    bf = sC[buf][ks * KSTEP + (lane >> 5)][k];
                }
                acc[i] = M::mma(a, bf, acc[i]);
            }
        }
        // grad_bias from the resident gO fragments, after the MFMA loop: a
        // branch between MFMAs would keep the B-fragment reads from being
        // issued ahead of them
        if constexpr (PREA) {
            if (do_bias) {
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
                    for (int e = 0; e < KPL; ++e) bsum += to_f32(a_set[buf][ks][e]);
            }
        }
    };

    // One step for tile t (the it-th of this work item, set S = it % 2).
    auto step = [&](auto s_c, int t) __attribute__((always_inline)) {
        constexpr int S = decltype(s_c)::value;
        constexpr int O = S ^ 1;
        if (t + 3 < t_end) load_om_tile(t + 3, om[O]);
        if (t + 1 < t_end && active) load_a_tile(a_set[O], t + 1);
        if (t + 2 < t_end) issue_tile(std::integral_constant<int, S>{}, t + 2, om[S]);
        mfma_tile(s_c, t);
        if (t + 1 < t_end) store_stage(std::integral_constant<int, O>{}, O);
        __syncthreads();
    };

    if (t_begin < t_end) {
        load_om_tile(t_begin, om[0]);
        if (t_begin + 1 < t_end) load_om_tile(t_begin + 1, om[1]);
        if (active) load_a_tile(a_set[0], t_begin);
        issue_tile(std::integral_constant<int, 0>{}, t_begin, om[0]);
        if (t_begin + 2 < t_end) load_om_tile(t_begin + 2, om[0]);
        if (t_begin + 1 < t_end) issue_tile(std::integral_constant<int, 1>{}, t_begin + 1, om[1]);
        store_stage(std::integral_constant<int, 0>{}, 0);
    }
    __syncthreads();
    // pairs of steps with no condition inside (a skipped second step would
    // give the loop head a second incoming path and the compiler's load
    // counting a conservative merge); an odd last tile is peeled
    int tt = t_begin;
    for (; tt + 1 < t_end; tt += 2) {
        step(std::integral_constant<int, 0>{}, tt);
        step(std::integral_constant<int, 1>{}, tt + 1);
    }
    if (tt < t_end) step(std::integral_constant<int, 0>{}, tt);

    if (!active) return;
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
        const int k = ch * KC + (kblk0 + i) * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = mc * 32 * MB + mblk * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m < p.Cout) unsafeAtomicAdd(p.gw_acc + (size_t)m * p.Kp + k, acc[i][r]);
        }
    }
    if (do_bias) {
        bsum += shfl_xor_f(bsum, 32);
        if (lane < 32 && mrow < p.Cout) unsafeAtomicAdd(p.gb_acc + mrow, bsum);
    }
}

// grad_weight for 2-byte types whose gO rows take 16-byte loads (N % 8 == 0,
// aligned base, at most kGoOutOfRange bytes per image): the work items,
// sampling pipeline and LDS stage of dcn2_gradw_kernel, with gO read in whole
// 128-byte lines.  The vector L1 looks up the lines of each group of
// consecutive lanes separately; loading the 32x32 A fragments directly (lane l
// = row l%32) touches a different line in every lane, 32 bytes of each.
// Instead load j = 4*lam + q (lam = 64-pixel line, q = 8-row group) gives
// lane l the 8-pixel chunk 8*lam + l%8 of row 8*q + l/8, so lanes 8g..8g+7
// read one whole line, and each wave passes its own 8 KB through LDS, chunk c
// of row r at 16-byte slot 17*r + c (the padding keeps both the stores and
// the reads of 8 consecutive lanes on distinct banks, and every address is a
// per-lane base plus a constant).  For K step i lane l reads chunk c = 2i +
// l/32 of row l%32: its A fragment, whose B fragment is LDS block c.  The
// loads of the next tile are stored at the end of the step that issued them
// (they have had its MFMA phase to land), so the MFMAs only wait for LDS
// reads, and one register set holds the loads in flight.  Rows past Cout and
// pixels past N read 0 (buffer range).
// Every stage runs unconditionally on a clamped tile index, so no load sits
// in a divergent branch and the compiler's count of outstanding loads stays
// exact across steps.
template <typename T, int MB, bool MASK, bool GN>
__global__ __launch_bounds__(512) void dcn2_gradw_line_kernel(const BwdParams p) {
    static_assert(sizeof(T) == 2, "2-byte types");
    using M = Mma<T>;
    using frag = typename M::frag;
    constexpr int KC = M::KC, KSTEP = M::KSTEP;
    constexpr int BN = 128, NKS = BN / KSTEP;
    constexpr int KB = KC / 32;
    constexpr int NBLK = MB * KB;
    constexpr int BPW = NBLK >= 16 ? 2 : 1;  // blocks per wave
    constexpr int CPS = KC / 4;
    static_assert(KSTEP == 16 && NKS == 8 && BN == 128, "8 K steps of 16 pixels: one 8x8 transpose");

    __shared__ __attribute__((aligned(16))) T sC[2][KC][BN];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int mblk, kblk0;
    if constexpr (BPW == 2) {
        mblk = wave;
        kblk0 = 0;
    } else {
        mblk = wave / KB;
        kblk0 = wave - mblk * KB;
    }
    // work item as in dcn2_gradw_kernel (every wave is active: NBLK >= 8)
    const int nmc = p.Mp / (32 * MB);
    const int wi = xcd_remap(blockIdx.x, p.splits * p.gw_nch * nmc);
    const int mc = wi % nmc, j = (wi / nmc) % p.gw_nch, sp = wi / (nmc * p.gw_nch);
    const int ch = gw_chunk(p, j, mc * 32 * MB);
    const bool do_bias = p.gb_acc != nullptr && j == 0 && kblk0 == 0;
    const int rbase = mc * 32 * MB + mblk * 32;  // first gO row of this wave
    const int mrow = rbase + (lane & 31);
    const int N = p.Ho * p.Wo, KK = p.kh * p.kw, cs = p.G * p.Cgp;
    const int T_total = p.B * p.tiles_per_img;
    const int t_begin = (int)((long)T_total * sp / p.splits);
    const int t_end = (int)((long)T_total * (sp + 1) / p.splits);

    SampleGeo sg;
    sg.H = p.H; sg.W = p.W; sg.kh = p.kh; sg.kw = p.kw; sg.sh = p.sh; sg.sw = p.sw;
    sg.ph = p.ph; sg.pw = p.pw; sg.dh = p.dh; sg.dw = p.dw; sg.G = p.G; sg.Cgp = p.Cgp;
    sg.Wo = p.Wo; sg.N = N; sg.cs = cs; sg.KK = KK; sg.msk_logit = p.msk_logit;
    const ChunkEnt cp = ((const ChunkEnt *)p.tab)[ch];
    // offset/mask loads 3 tiles ahead of the MFMA, corner gathers 2 ahead, the
    // column stage and the gO loads 1 ahead; sampler register sets by tile
    // parity (the loop is unrolled by two, so no register copies)
    Sampler<T, 1, MASK> smp[2];
    smp[0].init(tid);
    smp[1].init(tid);
    SlotOM<T, 1> om[2];

    auto load_om_tile = [&](int t, SlotOM<T, 1> &o) __attribute__((always_inline)) {
        const int b = t / p.tiles_per_img, n0 = (t - b * p.tiles_per_img) * BN;
        smp[0].load_om(n0, cp.x, sg, tid, (const T *)p.offset + (size_t)b * p.off_bs,
                       MASK ? (const T *)p.mask + (size_t)b * p.msk_bs : nullptr, o);
    };
    auto issue_tile = [&](auto set_c, int t, const SlotOM<T, 1> &o) __attribute__((always_inline)) {
        constexpr int set = decltype(set_c)::value;
        const int b = t / p.tiles_per_img;
        smp[set].issue(cp, sg, (const T *)p.xt + (size_t)b * p.H * p.W * cs, o);
    };
    auto store_stage = [&](auto set_c, int buf) __attribute__((always_inline)) {
        constexpr int set = decltype(set_c)::value;
        const int pl = tid >> 2;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            float v[8];
            smp[set].blend(0, u, v);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int k = smp[set].q * CPS + u * 8 + e;
                sC[buf][k][((pl >> 3) ^ gw_swz(k)) * 8 + (pl & 7)] = (T)v[e];
            }
        }
    };

    // one image's gO (the host keeps it within kGoOutOfRange bytes)
    const uint32_t go_bytes = (uint32_t)((size_t)p.Cout * N * sizeof(T));
    const int lg = lane >> 3, lc = lane & 7;
    uint4 ga[NKS];  // gO of the next tile, loaded by line; stored to LDS at the end of the step
    // NCHW: lanes 8g..8g+7 read one 128-byte line (8 pixels of a row) per
    // instruction.  Channels-last: lanes 4q..4q+3 read the wave's 32 channels
    // of one pixel (64 bytes), 16 pixels per instruction.
    auto load_a_tile = [&](uint4 (&a)[NKS], int t) __attribute__((always_inline)) {
        const int b = t / p.tiles_per_img, n0 = (t - b * p.tiles_per_img) * BN;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<T *>((const T *)p.gout + (size_t)b * p.Cout * N), (short)0, (int)go_bytes,
            0x00020000);
#pragma unroll
        for (int j = 0; j < NKS; ++j) {
            int off;
            if constexpr (GN) {
                const int n = n0 + 16 * j + (lane >> 2);
                const unsigned m = (unsigned)(rbase + 8 * (lane & 3));
                off = n < N && (int)m < p.Cout
                          ? (int)(((unsigned)n * (unsigned)p.Cout + m) * sizeof(T))
                          : kGoOutOfRange;
            } else {
                const unsigned row = (unsigned)(rbase + 8 * (j & 3) + lg);
                const int n = n0 + 64 * (j >> 2) + 8 * lc;
                off = n < N ? (int)((row * (unsigned)N + (unsigned)n) * sizeof(T)) : kGoOutOfRange;
            }
            a[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
        }
    };
    // Per-wave rearrangement area.  NCHW: 32 rows x 17 slots of 16 bytes, a
    // fragment is two 16-byte reads.  Channels-last: [128 pixels][32 rows],
    // a fragment (8 pixels of one row) is two transposing reads
    // (ds_read_b64_tr_b16: within 16 lanes, lane i receives element i%4 of
    // the 4-element pieces that lanes i/4, 4 + i/4, 8 + i/4, 12 + i/4 point
    // at; lane L points at 4 rows of pixel L/4, so lane i receives row i at
    // 4 consecutive pixels).
    __shared__ uint4 sG[8][32 * 17];
    uint4 *const gw_st = &sG[wave][17 * lg + lc];                     // + 17*8*q + 8*lam
    const uint4 *const gw_ld = &sG[wave][17 * (lane & 31) + (lane >> 5)];  // + 2*i
    T *const gn_base = reinterpret_cast<T *>(&sG[wave][0]);
    auto stash = [&]() __attribute__((always_inline)) {
        if constexpr (GN) {
#pragma unroll
            for (int j = 0; j < NKS; ++j) sG[wave][64 * j + lane] = ga[j];
        } else {
#pragma unroll
            for (int j = 0; j < NKS; ++j) gw_st[17 * 8 * (j & 3) + 8 * (j >> 2)] = ga[j];
        }
    };
    auto read_frag = [&](int ks) __attribute__((always_inline)) {
        if constexpr (GN) {
            typedef short s16x4 __attribute__((ext_vector_type(4)));
            const int g = lane >> 4, li = lane & 15;
            const int c0 = 16 * (g & 1) + 4 * (li & 3), p0 = ks * KSTEP + 8 * (g >> 1) + (li >> 2);
            s16x4 h[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
                h[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4 *)(gn_base + (p0 + 4 * hh) * 32 + c0));
            return __builtin_bit_cast(frag, __builtin_shufflevector(h[0], h[1], 0, 1, 2, 3, 4, 5, 6, 7));
        } else {
            return __builtin_bit_cast(frag, gw_ld[2 * ks]);
        }
    };

    f32x16 acc[BPW];
#pragma unroll
    for (int i = 0; i < BPW; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
    float bsum = 0.0f;

    auto mfma_tile = [&](auto s_c) __attribute__((always_inline)) {
        constexpr int buf = decltype(s_c)::value;
        frag af[NKS];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) af[ks] = read_frag(ks);
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            const frag a = af[ks];
#pragma unroll
            for (int i = 0; i < BPW; ++i) {
                const int k = (kblk0 + i) * 32 + (lane & 31);
                const int nblk = 2 * ks + (lane >> 5);
                const frag bf = *reinterpret_cast<const frag *>(&sC[buf][k][(nblk ^ gw_swz(k)) * 8]);
                acc[i] = M::mma(a, bf, acc[i]);
            }
        }
        // grad_bias from the resident fragments, after the MFMA loop (a branch
        // between MFMAs would keep the B-fragment reads from being issued
        // ahead of them)
        if (do_bias) {
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
                for (int e = 0; e < 8; ++e) bsum += to_f32(af[ks][e]);
            }
        }
    };

    const int t_last = t_end - 1;
    auto step = [&](auto s_c, int t) __attribute__((always_inline)) {
        constexpr int S = decltype(s_c)::value;
        constexpr int O = S ^ 1;
        load_om_tile(min(t + 3, t_last), om[O]);
        load_a_tile(ga, min(t + 1, t_last));
        issue_tile(std::integral_constant<int, S>{}, min(t + 2, t_last), om[S]);
        mfma_tile(s_c);
        store_stage(std::integral_constant<int, O>{}, O);
        stash();  // after this wave's reads of the current tile (LDS is in order per wave)
        __syncthreads();
    };

    if (t_begin < t_end) {
        load_om_tile(t_begin, om[0]);
        load_om_tile(min(t_begin + 1, t_last), om[1]);
        load_a_tile(ga, t_begin);
        issue_tile(std::integral_constant<int, 0>{}, t_begin, om[0]);
        load_om_tile(min(t_begin + 2, t_last), om[0]);
        issue_tile(std::integral_constant<int, 1>{}, min(t_begin + 1, t_last), om[1]);
        store_stage(std::integral_constant<int, 0>{}, 0);
        stash();
    }
    __syncthreads();
    // pairs of steps with no condition inside (a skipped second step would
    // give the loop head a second incoming path and the compiler's load
    // counting a conservative merge); an odd last tile is peeled
    int tt = t_begin;
    for (; tt + 1 < t_end; tt += 2) {
        step(std::integral_constant<int, 0>{}, tt);
        step(std::integral_constant<int, 1>{}, tt + 1);
    }
    if (tt < t_end) step(std::integral_constant<int, 0>{}, tt);

#pragma unroll
    for (int i = 0; i < BPW; ++i) {
        const int k = ch * KC + (kblk0 + i) * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = rbase + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m < p.Cout) unsafeAtomicAdd(p.gw_acc + (size_t)m * p.Kp + k, acc[i][r]);
        }
    }
    if (do_bias) {
        bsum += shfl_xor_f(bsum, 32);
        if (lane < 32 && mrow < p.Cout) unsafeAtomicAdd(p.gb_acc + mrow, bsum);
    }
}

// ---------------------------------------------------------------------------
// Fused backward kernel: column gradient, grad_offset / grad_mask, the
// grad_input hand-off, grad_weight and grad_bias in one pass over gO.  It
// serves 2-byte types with one 256-row M chunk (Mp == 256), one K chunk per
// deformable group (Cgp == KC) and gO rows that take 16-byte loads; other
// shapes run dcn2_colgrad_kernel and a grad_weight kernel.
//
// Grid: pixel-tile ranges x K chunks, one workgroup of 8 waves per CU (two
// per SIMD).  A workgroup keeps one K chunk, i.e. one (tap, group), and walks
// consecutive tiles of BN = 64 pixels.  Its grad_weight block gW[256][64] is
// accumulated in registers (rows 32w.. in wave w) over all of its tiles and
// added to the fp32 accumulator once.  Wave w owns K block kb = w%2 (32
// channels), pixel half P = (w/2)%2 and M half mh = w/4 of the column-gradient
// GEMM, whose W'^T fragments stay in its registers.  Each tile t takes two
// phases, with the tile's gO [256][64] and sampling descriptors in LDS and
// the wave's corner gathers in registers:
//   A  colgrad: partial cg[k][n] = sum over m in half mh of W'^T[k][m]
//      gO[m][n] for (kb, P) on MFMA -> LDS; between the MFMAs the next tile's
//      gO rows are loaded straight into the other LDS buffer.  The sampler
//      wave writes the next tile's descriptors (a lane per pixel); the
//      finisher wave turns the previous tile's corner sums into grad_offset /
//      grad_mask (a lane per pixel, as dcn2_colgrad_kernel does).
//   B  the next tile's corner gathers are loaded into the other register
//      set; consume: lane (pixel px0 + l/4, 8 channels of K block kb) adds the
//      two M halves' partials, then corner sums S_q = sum_c cg_c x_c(corner q)
//      over its channels, reduced over the pixel's 4 lanes -> LDS; the masked
//      cg row -> the sample's grad_input bucket row; the blended column ->
//      LDS.  Between these pieces the wave issues the MFMAs of the previous
//      tile's gW[m][k] += sum_n gO[m][n] col[k][n], so one wave's VALU runs
//      beside the other's MFMAs.
// The gO loads of a tile are waited for once, before its last barrier; the
// corner gathers and the sampler's offsets are waited for where they are
// used, a tile after they are issued.  A gather lane group of 4 lanes reads
// 64 contiguous bytes of one corner, so an instruction touches 16 cache
// lines.
//
// LDS layouts (16-byte pieces XOR-permuted per line so that the transposing
// 8-byte reads, the 16-byte reads and the 16-byte stores are free of bank
// conflicts; a wave's 1 KiB load lands on consecutive LDS bytes, so each lane
// loads the piece that belongs at its LDS slot):
//   NCHW gO          [256 rows m][64 pixels], piece j of row r at
//                    j ^ fused_swz(r); wave w loads rows 32w ...
//   channels-last gO [8 row blocks][64 pixels][32 rows], piece j (rows
//                    8j..8j+7 of the block) of pixel n at j ^ fused_swz_cl(n);
//                    wave w loads block w.
//   columns          [64 pixels][64 channels], piece j of pixel n at
//                    j ^ fused_swz_c(n), read as grad_weight B fragments by
//                    transposing reads.
//   cg partials      [M half][block (kb, P)][32 pixels][32 channels + 4].
__device__ __forceinline__ int fused_swz(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }
__device__ __forceinline__ int fused_swz_cl(int n) { return (((n >> 1) & 1) << 1) | ((n >> 2) & 1); }
__device__ __forceinline__ int fused_swz_c(int n) { return ((n & 3) << 1) | ((n >> 1) & 1); }

// Trash bytes each lane of the fused kernel may write (its widest hand-off row).
constexpr int kFusedTrashLane = 32;


template <typename T, bool GN, int MP>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void dcn2_bwd_fused_kernel(const BwdParams p) {
    static_assert(sizeof(T) == 2, "2-byte types");
    static_assert(MP == 256 || MP == 128, "128 or 256 padded output channels");
    using M = Mma<T>;
    using frag = typename M::frag;
    typedef typename RowOf<T>::type R;
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    constexpr int KC = M::KC, KSTEP = M::KSTEP;
    constexpr int BN = 64;
    constexpr int NMS = MP / KSTEP / 2;  // column-gradient MFMA steps of one M half
    constexpr int NKS = BN / KSTEP;      // grad_weight MFMA steps (over pixels)
    constexpr int RPW = MP / 8;          // gO rows each wave stages (32 or 16)
    constexpr int NGL = RPW / 8;         // its 1 KiB stage loads per tile (4 or 2)
    constexpr int NI = MP / 128;         // 32-column K blocks of a wave's grad_weight rows
    constexpr int LDX = 32 + 4;          // pitch (floats) of the cg areas
    constexpr int E = 8;                 // channels of one 16-byte piece
    constexpr int NST = E * (int)sizeof(R) / 16;  // 16-byte hand-off stores per lane
    static_assert(KC == 64 && Unpack<T>::E == E && NST * 16 <= kFusedTrashLane, "geometry");

    __shared__ __attribute__((aligned(16))) T sG[2][MP * BN];         // gO stage (double)
    __shared__ __attribute__((aligned(16))) float sX[2][4][32][LDX];  // cg partials [M half][block]
    __shared__ __attribute__((aligned(16))) T sC[2][BN][KC];          // blended columns (double)
    __shared__ __attribute__((aligned(16))) f32x4 sS[2][BN];          // corner sums per K block
    __shared__ __attribute__((aligned(16))) f32x4 sD[3][BN][3];       // sampling descriptors
    __shared__ int sV[3][BN];                                         // corner validity bits

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // column-gradient block (K block kb, pixels 32P..) and M half mh of this
    // wave; its gathered / consumed pixels are 32P + 16mh .. +15
    const int kb = wave & 1, P = (wave >> 1) & 1, mh = wave >> 2;
    const int blk = wave & 3, px0 = 32 * P + 16 * mh;
    // grad_weight block of this wave: rows gw_row0 .. +31 and the NI K blocks
    // from gw_i0 (MP 256: rows 32 wave, both K blocks; MP 128: rows
    // 32 (wave % 4), K block wave / 4)
    const int gw_row0 = MP == 256 ? 32 * wave : 32 * (wave & 3);
    const int gw_i0 = MP == 256 ? 0 : wave >> 2;
    const int N = p.Ho * p.Wo, KK = p.kh * p.kw, cs = p.G * p.Cgp;
    const int cpg = p.Cgp / KC;
    const int nch = KK * p.G * cpg;
    const int tpi = p.tiles_per_img;  // tiles of BN pixels per image
    // work item = (tile range sp, chunk c) with the chunk fastest, handed to
    // XCDs in contiguous ranges: the workgroups of one XCD share tile ranges,
    // so a gO tile is read from HBM about once per XCD
    const int wi = xcd_remap(blockIdx.x, p.splits * nch);
    const int c = wi % nch, sp = wi / nch;
    const int T_total = p.B * tpi;
    const int t_begin = (int)((long)T_total * sp / p.splits);
    const int t_end = (int)((long)T_total * (sp + 1) / p.splits);
    if (t_begin >= t_end) return;  // the whole workgroup
    const int t_last = t_end - 1;
    const ChunkEnt ce = ((const ChunkEnt *)p.tab)[c];
    const int plane = ce.x;  // offset / mask plane g*KK + tap
    // the chunk's first channel within its group's Cgp-wide hand-off row
    const int cbase = ce.w - (plane / KK) * p.Cgp;

    // W'^T fragments of K block kb, M half mh of chunk c (pack_weight_kernel
    // layout 1: fragment (row block 2c + kb, step s) is one contiguous run of
    // 64 lanes x 8 elements).
    frag wa[NMS];
    {
        const T *wrow = (const T *)p.wt + ((size_t)(c * (KC / 32) + kb) * (2 * NMS) + mh * NMS) * 512 +
                        lane * 8;
#pragma unroll
        for (int s = 0; s < NMS; ++s) wa[s] = *reinterpret_cast<const frag *>(wrow + s * 512);
    }

    // ---- gO stage --------------------------------------------------------
    // The wave's RPW gO rows of tile t (RPW * 128 bytes): load q (of NGL)
    // lands at LDS byte go_lds(buf) + 1024 q.  Rows past Cout and pixels past
    // N read zeros.
    auto go_lds = [&](int buf) __attribute__((always_inline)) {
        return lds_addr(&sG[buf][0]) + wave * (RPW * BN * (int)sizeof(T));
    };
    // Tile t = image b, pixels n0 .. n0 + BN - 1.
    struct TileId {
        int b, n0;
    };
    auto tile_id = [&](int t) __attribute__((always_inline)) {
        const int b = t / tpi;
        return TileId{b, (t - b * tpi) * BN};
    };
    const uint32_t go_bytes = (uint32_t)((size_t)p.Cout * N * sizeof(T));
    auto go_rsrc = [&](const TileId &id) __attribute__((always_inline)) {
        return __builtin_amdgcn_make_buffer_rsrc(
            const_cast<T *>((const T *)p.gout + (size_t)id.b * p.Cout * N), (short)0, (int)go_bytes,
            0x00020000);
    };
    // Load q of the wave's rows: NCHW rows RPW wave + 8q + l/8, 8 pieces of 8
    // pixels; channels-last 32-row block RPW wave / 32, pixel lines
    // (RPW wave % 32) * 2 + 16q + l/4, 4 pieces of 8 rows.  The per-lane part
    // of the byte offset (go_lo), the pixel of the piece within the tile
    // (go_px) and whether its row exists (go_ok).
    int go_lo[NGL], go_px[NGL];
    bool go_ok[NGL];
#pragma unroll
    for (int q = 0; q < NGL; ++q) {
        if constexpr (GN) {
            const int n = (RPW * wave % 32) * 2 + 16 * q + (lane >> 2);
            const int m = (RPW * wave / 32) * 32 + 8 * ((lane & 3) ^ fused_swz_cl(n));
            go_lo[q] = (n * p.Cout + m) * (int)sizeof(T);
            go_px[q] = n;
            go_ok[q] = m < p.Cout;
        } else {
            const int r = RPW * wave + 8 * q + (lane >> 3);
            const int n = 8 * ((lane & 7) ^ fused_swz(r));
            go_lo[q] = (r * N + n) * (int)sizeof(T);
            go_px[q] = n;
            go_ok[q] = r < p.Cout;
        }
    }
    auto go_off = [&](const TileId &id, int q) __attribute__((always_inline)) {
        const int hi = (GN ? id.n0 * p.Cout : id.n0) * (int)sizeof(T);
        return go_ok[q] && id.n0 + go_px[q] < N ? go_lo[q] + hi : kGoOutOfRange;
    };
    // NCHW: element (row r, pixel x); channels-last: element (pixel n, row m);
    // columns: element (pixel n, channel k)
    auto at_rm = [&](int buf, int r, int x) __attribute__((always_inline)) {
        return &sG[buf][r * BN + (((x >> 3) ^ fused_swz(r)) << 3) + (x & 7)];
    };
    auto at_nm = [&](int buf, int n, int m) __attribute__((always_inline)) {
        return &sG[buf][(m >> 5) * (BN * 32) + n * 32 + ((((m >> 3) & 3) ^ fused_swz_cl(n)) << 3) +
                        (m & 7)];
    };
    auto at_c = [&](int cb, int n, int k) __attribute__((always_inline)) {
        return &sC[cb][n][(((k >> 3) ^ fused_swz_c(n)) << 3) + (k & 7)];
    };
    // Transposing read (ds_read_b64_tr_b16: within 16 lanes, lane i receives
    // element i%4 of the 4-element pieces that lanes i/4, 4 + i/4, 8 + i/4,
    // 12 + i/4 point at).  Lane L of 16-lane group g points at 4 consecutive
    // elements of line (l0 + 8*(g>>1) + 4*hh + L/4), starting at element
    // x0 + 16*(g&1) + 4*(L%4) of the line; lane l then holds element
    // x0 + l%32 of lines l0 + 8*(l/32) .. +7: an MFMA fragment whose 8 K
    // values run across the lines.
    auto tr_frag = [&](auto addr, int l0, int x0) __attribute__((always_inline)) {
        const int g = lane >> 4, li = lane & 15;
        s16x4 h[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
            h[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4 *)addr(
                    l0 + 8 * (g >> 1) + 4 * hh + (li >> 2), x0 + 16 * (g & 1) + 4 * (li & 3)));
        return __builtin_bit_cast(frag, __builtin_shufflevector(h[0], h[1], 0, 1, 2, 3, 4, 5, 6, 7));
    };
    // Column-gradient B fragment of M step s (0..15): gO rows 16s + 8*(l/32)
    // .., pixel 32P + l%32.  grad_weight A fragment of step ks: row
    // 32 wave + l%32, pixels 16 ks + 8*(l/32) ...
    auto go_bfrag = [&](int buf, int s) __attribute__((always_inline)) {
        if constexpr (GN) {
            return *reinterpret_cast<const frag *>(
                at_nm(buf, P * 32 + (lane & 31), s * KSTEP + 8 * (lane >> 5)));
        } else {
            return tr_frag([&](int r, int x) { return at_rm(buf, r, x); }, s * KSTEP, P * 32);
        }
    };
    auto go_afrag = [&](int buf, int ks) __attribute__((always_inline)) {
        if constexpr (GN) {
            return tr_frag([&](int n, int m) { return at_nm(buf, n, m); }, ks * KSTEP, gw_row0);
        } else {
            return *reinterpret_cast<const frag *>(
                at_rm(buf, gw_row0 + (lane & 31), ks * KSTEP + 8 * (lane >> 5)));
        }
    };

    // ---- sampling: wave kSampler, one lane per pixel of the tile ------------
    // Offsets, mask and bucket row of a tile's pixel `lane`, loaded a tile
    // before they are used and kept raw (no instruction reads them until
    // then, so their load is never waited for early).
    constexpr int kSampler = 1, kFinisher = 0;
    struct OM {
        T dy, dx, m;
        int sx;
    };
    auto load_om = [&](const TileId &id, OM &o) __attribute__((always_inline)) {
        const int b = id.b;
        const int nr = id.n0 + lane;
        const int nn = nr < N ? nr : 0;
        const T *offs = (const T *)p.offset + (size_t)b * p.off_bs + (size_t)plane * 2 * N;
        // (without a mask the load re-reads the offset: no load in a branch)
        const T *mk = p.mask ? (const T *)p.mask + (size_t)b * p.msk_bs + (size_t)plane * N : offs;
        o.dy = offs[nn];
        o.dx = offs[N + nn];
        o.m = mk[nn];
        o.sx = p.sidx[((size_t)b * p.G * KK + plane) * N + nn];
    };
    // Output row and column of the sampler lane's pixel in tile t, kept
    // incrementally (tiles of one workgroup are consecutive): sample() is
    // called for t_begin, t_begin + 1, ... in order.
    int s_t = -2, s_oy = 0, s_ox = 0;  // (s_t: the tile last sampled; none yet)
    auto advance_pixel = [&](int t, int n0) __attribute__((always_inline)) {
        if (t != s_t + 1 || n0 == 0) {  // first tile, or a new image
            const int nr = n0 + lane;
            s_oy = nr / p.Wo;
            s_ox = nr - s_oy * p.Wo;
        } else {
            s_ox += BN;
            while (s_ox >= p.Wo) {
                s_ox -= p.Wo;
                ++s_oy;
            }
        }
        s_t = t;
    };
    // Descriptors of tile t's pixel `lane` into sD[buf][lane] (corner
    // weights; mask value, bucket row, fractions; corner element offsets) and
    // sV[buf][lane] (corner validity).
    auto sample = [&](int t, const TileId &id, const OM &o, int buf) __attribute__((always_inline)) {
        advance_pixel(t, id.n0);
        const int nr = id.n0 + lane;
        const bool live = nr < N;
        const float y = (float)(s_oy * p.sh - p.ph + ce.y) + to_f32(o.dy);
        const float x = (float)(s_ox * p.sw - p.pw + ce.z) + to_f32(o.dx);
        float mv = p.mask ? to_f32(o.m) : 1.0f;
        if (p.msk_logit) mv = mask_value(mv, 1);
        mv = live ? mv : 0.0f;
        const SamplePos spos = sample_pos(live ? y : -2.0f, live ? x : -2.0f, p.H, p.W);
        const Corners cr = make_corners(spos, mv, p.W, cs);
        sD[buf][lane][0] = f32x4{cr.w[0], cr.w[1], cr.w[2], cr.w[3]};
        sD[buf][lane][1] = f32x4{mv, __int_as_float(live ? o.sx : -1), spos.ly, spos.lx};
        sD[buf][lane][2] = f32x4{__int_as_float(cr.off[0]), __int_as_float(cr.off[1]),
                                 __int_as_float(cr.off[2]), __int_as_float(cr.off[3])};
        sV[buf][lane] = (spos.vy0 && spos.vx0 ? 1 : 0) | (spos.vy0 && spos.vx1 ? 2 : 0) |
                        (spos.vy1 && spos.vx0 ? 4 : 0) | (spos.vy1 && spos.vx1 ? 8 : 0);
    };
    // Corner gathers of the wave's pixels px0 .. px0+15: load q brings corner
    // q, lanes 4i..4i+3 the 64 bytes (32 channels of K block kb) of pixel
    // px0 + i; the corner offsets come from the descriptors in sD[buf].
    auto gather_offsets = [&](int buf) __attribute__((always_inline)) {
        return sD[buf][px0 + (lane >> 2)][2];
    };
    // (one image of xt is below 2 GiB: 32-bit byte offsets)
    const uint32_t xt_bytes = (uint32_t)((size_t)p.H * p.W * cs * sizeof(T));
    auto xt_rsrc = [&](const TileId &id) __attribute__((always_inline)) {
        return __builtin_amdgcn_make_buffer_rsrc(
            const_cast<T *>((const T *)p.xt + (size_t)id.b * p.H * p.W * cs), (short)0, (int)xt_bytes,
            0x00020000);
    };
    const int gather_lane = (ce.w + kb * 32 + (lane & 3) * E) * (int)sizeof(T);
    auto gather_off = [&](int q, const f32x4 &goff) __attribute__((always_inline)) {
        return __float_as_int(goff[q]) * (int)sizeof(T) + gather_lane;
    };
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    // the lane's corner gathers of tile t (load q: corner q) into registers
    auto gather = [&](const __amdgpu_buffer_rsrc_t &xrs, const f32x4 &goff, uint4 (&raw)[4])
        __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xrs, gather_off(q, goff), 0, 0);
            raw[q] = make_uint4(v.x, v.y, v.z, v.w);
        }
    };

    // this lane's kFusedTrashLane bytes of dcn2_trash
    constexpr int kTrashWaves = kTrashBytes / (64 * kFusedTrashLane);
    uint4 *const trash_v = reinterpret_cast<uint4 *>(dcn2_trash) +
                           ((blockIdx.x * 8 + wave) % kTrashWaves) * (64 * kFusedTrashLane / 16) +
                           lane * (kFusedTrashLane / 16);
    T *const trash_t = reinterpret_cast<T *>(trash_v);

    // ---- phase A: column gradient ---------------------------------------------
    // Partial cg of block (kb, P) over the wave's M half -> sX[mh][blk].
    // after(s) runs after MFMA s (it issues the next tile's gO loads).  The
    // fragments are read two steps ahead; each step ends in a scheduling
    // barrier, which keeps that order and the loads where they are.
    auto colgrad = [&](int buf, auto after) __attribute__((always_inline)) {
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
        frag bf[NMS];
        bf[0] = go_bfrag(buf, mh * NMS);
        bf[1] = go_bfrag(buf, mh * NMS + 1);
#pragma unroll
        for (int s = 0; s < NMS; ++s) {
            if (s + 2 < NMS) bf[s + 2] = go_bfrag(buf, mh * NMS + s + 2);
            acc = M::mma(wa[s], bf[s], acc);
            after(s);
            __builtin_amdgcn_sched_barrier(0);
        }
        // acc[r] = cg[32kb + 8(r/4) + 4(l/32) + r%4][32P + l%32]
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<f32x4 *>(&sX[mh][blk][lane & 31][8 * j + 4 * (lane >> 5)]) =
                f32x4{acc[4 * j], acc[4 * j + 1], acc[4 * j + 2], acc[4 * j + 3]};
    };
    // Lane (pixel px0 + l/4, channels 32kb + 8(l%4) ..): corner sums, hand-off
    // and blend.  raw: the lane's corner gathers (read before the barrier).
    // between(j), j = 0..7, runs at eight points of the work, each fenced by
    // scheduling barriers (it issues the MFMAs that overlap this VALU work).
    const int pq = lane >> 2, cq = lane & 3;
    auto consume = [&](int buf, int dbuf, const uint4 (&raw)[4], auto between) __attribute__((always_inline)) {
        auto at = [&](int j) __attribute__((always_inline)) {
            __builtin_amdgcn_sched_barrier(0);
            between(j);
            __builtin_amdgcn_sched_barrier(0);
        };
        const int px = px0 + pq;
        const f32x4 d0 = sD[dbuf][px][0], d1 = sD[dbuf][px][1];
        float cgv[E];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(&sX[0][blk][16 * mh + pq][cq * E + 4 * h]) +
                            *reinterpret_cast<const f32x4 *>(&sX[1][blk][16 * mh + pq][cq * E + 4 * h]);
#pragma unroll
            for (int e = 0; e < 4; ++e) cgv[4 * h + e] = v[e];
        }
        at(0);
        // corner sums over the lane's 8 channels, then over the 4 lanes of the
        // pixel.  f16: 2-element dot products (v_dot2_f32_f16) of the corner
        // values with the column gradient rounded to f16, accumulated in fp32
        // (the rounding is that of the f16 grad_offset / grad_mask outputs).
        f32x4 S;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float s = 0.0f;
            if constexpr (std::is_same<T, f16>::value) {
                typedef f16 h2 __attribute__((ext_vector_type(2)));
                typedef float f2 __attribute__((ext_vector_type(2)));
                const f16x8 x = __builtin_bit_cast(f16x8, raw[q]);
#pragma unroll
                for (int e = 0; e < E / 2; ++e) {
                    const h2 cg2 = __builtin_convertvector(f2{cgv[2 * e], cgv[2 * e + 1]}, h2);
                    s = __builtin_amdgcn_fdot2(cg2, h2{x[2 * e], x[2 * e + 1]}, s, false);
                }
            } else {
                float v[E];
                Unpack<T>::run(raw[q], v);
#pragma unroll
                for (int e = 0; e < E; ++e) s = fmaf(cgv[e], v[e], s);
            }
            s += quad_xor1(s);
            s += quad_xor2(s);
            S[q] = s;
            if (q < 3) at(1 + q);
        }
        if (cq == 0) sS[kb][px] = S;
        at(4);
        // masked column-gradient row
        {
            const int srow = __float_as_int(d1[1]);
            float mrow[E];
#pragma unroll
            for (int e = 0; e < E; ++e) mrow[e] = cgv[e] * d1[0];
            uint4 *row = srow >= 0
                             ? reinterpret_cast<uint4 *>((R *)p.cgm + (size_t)srow * p.Cgp + cbase + kb * 32 +
                                                         cq * E)
                             : trash_v;
            if constexpr (kRowScaled<T>) {
                // the pixel's quad of lanes holds 32-channel block kb of the row
                unsigned code;
                const float f = row_block_scale(mrow, code);
#pragma unroll
                for (int e = 0; e < E; ++e) mrow[e] *= f;
                unsigned char *sc = srow >= 0 && cq == 0
                                        ? p.rsc + (size_t)srow * (p.Cgp / 32) + cbase / 32 + kb
                                        : reinterpret_cast<unsigned char *>(trash_v) + 8;
                *sc = (unsigned char)code;
            }
#pragma unroll
            for (int u = 0; u < NST; ++u) row[u] = pack16<R>(mrow + u * (16 / sizeof(R)));
        }
        at(5);
        // blended columns
        {
            float col[E], v[E];
#pragma unroll
            for (int e = 0; e < E; ++e) col[e] = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                Unpack<T>::run(raw[q], v);
#pragma unroll
                for (int e = 0; e < E; ++e) col[e] = fmaf(d0[q], v[e], col[e]);
                if (q == 1) at(6);
            }
            *reinterpret_cast<uint4 *>(at_c(buf, px, kb * 32 + cq * E)) = pack16<T>(col);
        }
        at(7);
    };

    // ---- phase B ----------------------------------------------------------------
    // grad_mask / grad_offset of pixel `lane` of tile t from both K blocks'
    // corner sums (wave kFinisher; pixels past N store to dcn2_trash).
    auto finish_sums = [&](int buf, const TileId &id) __attribute__((always_inline)) {
        const int b = id.b;
        const int nr = id.n0 + lane;
        const f32x4 S = sS[0][lane] + sS[1][lane];
        if (cpg > 1) {
            // a group of several chunks: this chunk's part of the corner sums
            // goes to p.csum, summed over the group's chunks there, and
            // ring_final_kernel (corner_finish) turns the totals into grad_offset /
            // grad_mask
            float *cs4 = p.csum + (((size_t)b * p.G * KK + plane) * N + (nr < N ? nr : 0)) * 4;
            if (nr < N) {
#pragma unroll
                for (int q = 0; q < 4; ++q) unsafeAtomicAdd(cs4 + q, S[q]);
            }
            return;
        }
        const f32x4 d1 = sD[buf][lane][1];
        const int valid = sV[buf][lane];
        const float mv = d1[0], fly = d1[2], flx = d1[3];
        const float S0 = (valid & 1) ? S[0] : 0.0f, S1 = (valid & 2) ? S[1] : 0.0f;
        const float S2 = (valid & 4) ? S[2] : 0.0f, S3 = (valid & 8) ? S[3] : 0.0f;
        const float hy = 1.0f - fly, hx = 1.0f - flx;
        const float goy = mv * (hx * (S2 - S0) + flx * (S3 - S1));
        const float gox = mv * (hy * (S1 - S0) + fly * (S3 - S2));
        const float gmr = hy * hx * S0 + hy * flx * S1 + fly * hx * S2 + fly * flx * S3;
        // d/d(logit) of sigmoid = s (1 - s), s = the mask value used
        const float gm = p.msk_logit ? gmr * mv * (1.0f - mv) : gmr;
        const bool live = nr < N;
        T *go = (T *)p.goff + (size_t)b * p.off_bs + (size_t)plane * 2 * N + nr;
        *(live ? go : trash_t) = from_f32<T>(goy);
        *(live ? go + N : trash_t + 1) = from_f32<T>(gox);
        T *gmp = p.gmask ? (T *)p.gmask + (size_t)b * p.msk_bs + (size_t)plane * N + nr : trash_t + 2;
        *(live ? gmp : trash_t + 2) = from_f32<T>(gm);
    };
    f32x16 gacc[NI];  // gW rows gw_row0 .., K blocks gw_i0 ..
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) gacc[i][r] = 0.0f;
    float bsum = 0.0f;
    // (grad_bias once per row: from chunk 0, by the waves of K block 0)
    const bool do_bias = p.gb_acc != nullptr && c == 0 && gw_i0 == 0;
    // acc + the sum of a fragment's 8 values (four 2-element dot products
    // with (1, 1), accumulated in fp32)
    auto sum8 = [](frag a, float acc) __attribute__((always_inline)) {
        typedef T t2 __attribute__((ext_vector_type(2)));
        const t2 one = {(T)1.0f, (T)1.0f};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const t2 pr2 = {a[2 * e], a[2 * e + 1]};
            if constexpr (std::is_same<T, f16>::value)
                acc = __builtin_amdgcn_fdot2(pr2, one, acc, false);
            else
                acc = __builtin_amdgcn_fdot2_f32_bf16(pr2, one, acc, false);
        }
        return acc;
    };
    // grad_weight A fragments of the wave's own gO rows (rows 32 wave ..,
    // which only this wave loads) of the tile in sG[buf]
    auto read_afrags = [&](int buf, frag (&a)[NKS]) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) a[ks] = go_afrag(buf, ks);
    };
    // grad_weight B fragments (columns of the tile in sC[cb]) and MFMA j =
    // 2 ks + i of gW += gO cols^T (grad_bias: compile-time switch, so no
    // branch sits between the MFMAs)
    auto read_bfrags = [&](int cb, frag (&b)[NKS][NI]) __attribute__((always_inline)) {
        const auto atc = [&](int n, int k) __attribute__((always_inline)) { return at_c(cb, n, k); };
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
            for (int i = 0; i < NI; ++i) b[ks][i] = tr_frag(atc, ks * KSTEP, (gw_i0 + i) * 32);
    };
    // MFMA point j (0 .. 2 NKS - 1) of a tile's grad_weight: MP 256 runs one
    // MFMA at every point (j = 2 ks + i), MP 128 one at every even point
    auto gradw_mma = [&](const frag (&a)[NKS], const frag (&b)[NKS][NI], int j, auto bias_c)
        __attribute__((always_inline)) {
        if (NI == 1 && (j & 1)) return;
        const int ks = j >> 1, i = NI == 2 ? (j & 1) : 0;
        gacc[i] = M::mma(a[ks], b[ks][i], gacc[i]);
        if constexpr (decltype(bias_c)::value)
            if (i == NI - 1) bsum = sum8(a[ks], bsum);
    };
    auto gradw = [&](const frag (&a)[NKS], int cb, auto bias_c) __attribute__((always_inline)) {
        frag b[NKS][NI];
        read_bfrags(cb, b);
#pragma unroll
        for (int j = 0; j < 2 * NKS; ++j) gradw_mma(a, b, j, bias_c);
    };

    // ---- the tiles ----------------------------------------------------------------
    // Two phases per tile t, one barrier after each:
    //   A  column gradient of t (MFMA) -> sX, with t+1's gO rows loaded
    //      between the MFMAs; the wave's corner gathers of t read from LDS;
    //      the sampler writes t+1's descriptors; the finisher turns t-1's
    //      corner sums into grad_offset / grad_mask.
    //   B  t+1's corner gathers are loaded into the wave's gather area;
    //      consume(t) (VALU: corner sums, hand-off, blend -> sC[t % 2]) runs
    //      beside grad_weight of t-1 (MFMA, columns from sC[(t - 1) % 2]), so
    //      one wave's VALU overlaps the other's MFMAs; then the wave reads
    //      t's grad_weight A fragments from its own gO rows into registers.
    // gO: double-buffered; a buffer is reloaded (in phase A of t+1) only with
    // the rows of the waves that already hold its A fragments, which each
    // wave reads from its own rows only.  Columns: double-buffered.
    // Descriptors: three buffers, tile t's in sD[(t - t_begin) % 3] (written
    // in phase A of t-1, read until phase A of t+1).  Everything a tile loads
    // is waited for once, before its last barrier.  The sampler's offsets of
    // tile t+1 are loaded at the top of tile t-1 into the register set of
    // tile t+1's parity (the loop is unrolled by two), so the end-of-tile wait
    // has covered them when they are used and no register copy or early wait
    // is needed.
    auto tiles = [&](auto bias_c) __attribute__((always_inline)) {
        OM om[2];
        uint4 rawset[2][4];  // corner gathers of the tiles of either parity
        const TileId id0 = tile_id(t_begin);
        if (wave == kSampler) {
            load_om(id0, om[0]);
            sample(t_begin, id0, om[0], 0);
            load_om(tile_id(min(t_begin + 1, t_last)), om[1]);
        }
        __syncthreads();  // descriptors of the first tile
        {
            const f32x4 goff = gather_offsets(0);
            const __amdgpu_buffer_rsrc_t grs = go_rsrc(id0), xrs = xt_rsrc(id0);
#pragma unroll
            for (int q = 0; q < NGL; ++q) dma16(grs, go_off(id0, q), go_lds(0) + q * 1024);
            gather(xrs, goff, rawset[0]);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the stage loads
        __syncthreads();
        int d3 = 0;    // (t - t_begin) % 3
        frag ga[NKS];  // grad_weight A fragments of the previous tile
        // tile t, buffer parity `buf` = (t - t_begin) % 2; `first`: t == t_begin
        auto step = [&](auto buf_c, auto first_c, int t) __attribute__((always_inline)) {
            constexpr int buf = decltype(buf_c)::value;
            constexpr bool first = decltype(first_c)::value;
            const int d3n = d3 == 2 ? 0 : d3 + 1, d3p = d3 == 0 ? 2 : d3 - 1;
            const int tn = min(t + 1, t_last);
            const TileId itn = tile_id(tn);
            if (wave == kSampler)  // tile t+2 has t's parity
                load_om(tile_id(min(t + 2, t_last)), om[buf]);
            // phase A
            {
                const __amdgpu_buffer_rsrc_t grs = go_rsrc(itn);
                const unsigned gl = go_lds(buf ^ 1);
                colgrad(buf, [&](int s) __attribute__((always_inline)) {
                    if (s & 1) dma16(grs, go_off(itn, s >> 1), gl + (s >> 1) * 1024);
                });
            }
            if (wave == kSampler) sample(tn, itn, om[buf ^ 1], d3n);
            if constexpr (!first)
                if (wave == kFinisher) finish_sums(d3p, tile_id(t - 1));
            __syncthreads();  // cg partials of both M halves; tile t+1's descriptors
            // phase B
            // tile t+1's corner gathers into the other register set: nothing
            // waits for them before tile t+1's phase B
            gather(xt_rsrc(itn), gather_offsets(d3n), rawset[buf ^ 1]);
            frag gb[NKS][NI];
            if constexpr (!first) read_bfrags(buf ^ 1, gb);
            consume(buf, d3, rawset[buf], [&](int j) __attribute__((always_inline)) {
                if constexpr (!first) gradw_mma(ga, gb, j, bias_c);
            });
            read_afrags(buf, ga);
            // The next tile's gO rows were loaded in phase A, before its four
            // corner gathers and the NST hand-off stores of consume():
            // waiting until at most 4 + NST memory operations are outstanding
            // waits for the gO rows and leaves the gathers and stores in flight.
            __builtin_amdgcn_s_waitcnt(0x0F70 | (4 + NST));
            __syncthreads();  // sums, columns, the next tile's gO rows and gathers
            d3 = d3n;
        };
        // the first tile peeled, then pairs of steps with no condition inside;
        // an odd last tile is peeled
        step(std::integral_constant<int, 0>{}, std::true_type{}, t_begin);
        int t = t_begin + 1;
        for (; t + 1 < t_end; t += 2) {
            step(std::integral_constant<int, 1>{}, std::false_type{}, t);
            step(std::integral_constant<int, 0>{}, std::false_type{}, t + 1);
        }
        if (t < t_end) step(std::integral_constant<int, 1>{}, std::false_type{}, t);
        // the last tile's grad_offset / grad_mask and grad_weight
        const int db = d3 == 0 ? 2 : d3 - 1;  // the last tile's descriptors
        if (wave == kFinisher) finish_sums(db, tile_id(t_last));
        gradw(ga, (t_last - t_begin) & 1, bias_c);
    };
    if (do_bias) tiles(std::true_type{});
    else tiles(std::false_type{});

    // grad_weight block of this wave: rows gw_row0 .., columns c*KC + 32 (gw_i0 + i) ..
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int k = c * KC + (gw_i0 + i) * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = gw_row0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m < p.Cout) unsafeAtomicAdd(p.gw_acc + (size_t)m * p.Kp + k, gacc[i][r]);
        }
    }
    if (do_bias) {
        const float v = bsum + shfl_xor_f(bsum, 32);
        const int m = gw_row0 + (lane & 31);
        if (lane < 32 && m < p.Cout) unsafeAtomicAdd(p.gb_acc + m, v);
    }
}

// ---------------------------------------------------------------------------
// grad_offset / grad_mask of the fused kernel for groups of several channel
// chunks: the corner sums S_q of a sample, summed over the group's chunks in
// csum by the fused kernel's workgroups, become the coordinate and mask
// gradients (com.cu:431-501), with the sample position, corner validity and
// mask value recomputed from the offsets exactly as the fused kernel's
// sampler does.  One thread per sample (pixel n, plane g*KK + tap, image b),
// run as a block range of ring_final_kernel.
template <typename T>
__device__ __forceinline__ void corner_finish(const BwdParams &p, int n, int plane, int b) {
    const int N = p.Ho * p.Wo, KK = p.kh * p.kw;
    const int tap = plane % KK, ki = tap / p.kw, kj = tap - ki * p.kw;
    const int oy = n / p.Wo, ox = n - oy * p.Wo;
    const T *offs = (const T *)p.offset + (size_t)b * p.off_bs + (size_t)plane * 2 * N;
    const float y = (float)(oy * p.sh - p.ph + ki * p.dh) + to_f32(offs[n]);
    const float x = (float)(ox * p.sw - p.pw + kj * p.dw) + to_f32(offs[N + n]);
    float mv = 1.0f;
    if (p.mask) {
        mv = to_f32(((const T *)p.mask)[(size_t)b * p.msk_bs + (size_t)plane * N + n]);
        if (p.msk_logit) mv = mask_value(mv, 1);
    }
    const SamplePos sp = sample_pos(y, x, p.H, p.W);
    const f32x4 S = *reinterpret_cast<const f32x4 *>(p.csum + (((size_t)b * p.G * KK + plane) * N + n) * 4);
    const float S0 = sp.vy0 && sp.vx0 ? S[0] : 0.0f, S1 = sp.vy0 && sp.vx1 ? S[1] : 0.0f;
    const float S2 = sp.vy1 && sp.vx0 ? S[2] : 0.0f, S3 = sp.vy1 && sp.vx1 ? S[3] : 0.0f;
    const float fly = sp.ly, flx = sp.lx, hy = 1.0f - fly, hx = 1.0f - flx;
    const float goy = mv * (hx * (S2 - S0) + flx * (S3 - S1));
    const float gox = mv * (hy * (S1 - S0) + fly * (S3 - S2));
    const float gmr = hy * hx * S0 + hy * flx * S1 + fly * hx * S2 + fly * flx * S3;
    const float gm = p.msk_logit ? gmr * mv * (1.0f - mv) : gmr;
    T *go = (T *)p.goff + (size_t)b * p.off_bs + (size_t)plane * 2 * N + n;
    go[0] = from_f32<T>(goy);
    go[N] = from_f32<T>(gox);
    if (p.gmask) ((T *)p.gmask)[(size_t)b * p.msk_bs + (size_t)plane * N + n] = from_f32<T>(gm);
}

// ---------------------------------------------------------------------------
// grad_input gather.  One block per bucket (image, group, 16x16 cell tile).
// The bucket's records are taken in batches of up to kGatherBatch; each
// batch is counting-sorted by cell in LDS, together with the fractional
// sample coordinates.  Then every pixel of the (TS+1)^2 window the tile's
// corners can reach is pulled by one lane group (lane = channel): pixel
// (py, px) is corner 00 of cell (py, px), 01 of (py, px-1), 10 of (py-1, px)
// and 11 of (py-1, px-1), so its value is the sum over the batch's records of
// those four cells of (bilinear corner weight) x (masked column-gradient
// row), computed in a register with up to two batches of row loads in
// flight.  Interior pixels (reachable from this tile's cells only) are final
// after the bucket's last batch: they are staged in LDS in the caller's type
// and written straight to grad_input in its layout (a bucket of several
// batches keeps their partial sums in gi_acc between batches).  The sums of
// the one-pixel border ring, shared with the neighbouring tiles, are stored
// per bucket (kRing pixels; the first batch stores, later batches add), and
// ring_final_kernel, launched after this kernel, writes every tile-boundary
// pixel of grad_input from the rings that hold it.  Every entry of the ring
// is written on every call, an empty bucket's included.  This replaces the
// global atomic per (sample, corner, channel) of the reference's col2im
// scatter (com.cu:553-609) with plain stores.
constexpr int kGatherBatch = 4096;  // records of one batch the LDS sort holds
// Buffer offset past one batch's rows (the host keeps kGatherBatch * Cgp * esz
// below it), so a load there reads 0.
constexpr int kGatherOutOfRange = 0x7ffffff0;
// static LDS of dcn2_gi_gather_kernel: cell counts and starts, sorted slots and fractions,
// each wave's 8 pixels of grad_input for the NCHW write-out (one channel chunk of 128
// bytes per pixel), plus the sorted scale codes of bf16 rows
constexpr int kGatherStaticLds = kCellTile * kCellTile * 4 + (kCellTile * kCellTile + 1) * 4 +
                                 kGatherBatch * 2 + kGatherBatch * 8 + 8 * 8 * 128;
constexpr int gather_static_lds(bool scaled) { return kGatherStaticLds + (scaled ? kGatherBatch * 2 : 4); }

template <typename T>
__global__ __launch_bounds__(512) void dcn2_gi_gather_kernel(const BwdParams p) {
    constexpr int KC = Mma<T>::KC;  // channels per pass
    constexpr int TS = kCellTile, TW = TS + 1, NCELL = TS * TS;
    constexpr int RPT = kGatherBatch / 512;
    __shared__ int ccnt[NCELL];
    __shared__ int cstart[NCELL + 1];
    __shared__ unsigned short sslot[kGatherBatch];    // row in the batch, sorted by cell
    __shared__ float2 sfrac[kGatherBatch];            // (ly, lx), sorted by cell
    __shared__ unsigned short ssc[kRowScaled<T> ? kGatherBatch : 2];  // bf16 rows: the chunk's scale codes
    // each wave's 8 pixels of one channel chunk, transposed for the NCHW write-out
    __shared__ __attribute__((aligned(16))) T stage[8][8 * KC];
    static_assert(sizeof(ccnt) + sizeof(cstart) + sizeof(sslot) + sizeof(sfrac) + sizeof(ssc) +
                          sizeof(stage) ==
                      gather_static_lds(kRowScaled<T>),
                  "the launch's occupancy cap assumes this static LDS");
    static_assert(KC * sizeof(T) == 128, "one channel chunk of a pixel is 128 bytes");

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nb = p.B * p.G * p.nty * p.ntx;
    const int bucket = xcd_remap(blockIdx.x, nb);
    const int tx = bucket % p.ntx, ty = (bucket / p.ntx) % p.nty;
    const int bg = bucket / (p.ntx * p.nty), b = bg / p.G, g = bg - b * p.G;
    const int row0 = p.bstart[bucket], count = p.bstart[bucket + 1] - row0;
    const int oy = ty * TS - 1, ox = tx * TS - 1;  // pixel of local (0, 0)
    const int cpg = p.Cgp / KC;
    // A bucket of several batches (count > kGatherBatch) keeps its interior
    // pixels' partial sums between batches in its gi_acc slot
    // [(TS-1)^2 pixels][Cgp], slot row0 / (kGatherBatch + 1): the row ranges of
    // two such buckets start at least kGatherBatch + 1 rows apart, so no two
    // share a slot.
    float *__restrict__ gi =
        p.gi_acc + (size_t)(row0 / (kGatherBatch + 1)) * (TS - 1) * (TS - 1) * p.Cgp;

    // one pass per batch of records; an empty bucket still takes one (with no
    // records) to write its ring
    for (int base = 0; base == 0 || base < count; base += kGatherBatch) {
        const int nrec = min(count - base, kGatherBatch);
        const BucketRec *__restrict__ recs = p.rec + (size_t)row0 + base;
        const bool first = base == 0, last = base + kGatherBatch >= count;
        if (!first) __syncthreads();  // the previous batch is done with the LDS arrays

        // 1. counting sort by cell (cell = local row * TS + local column)
        for (int i = tid; i < NCELL; i += 512) ccnt[i] = 0;
        __syncthreads();
        int key[RPT];  // (cell << 16) | rank, or -1
        float2 fr[RPT];
#pragma unroll
        for (int k = 0; k < RPT; ++k) {
            const int r = tid + k * 512;
            key[k] = -1;
            fr[k] = make_float2(0.f, 0.f);
            if (r < nrec) {
                const BucketRec rc = recs[r];
                const int cy = (int)(short)(rc.yx & 0xffff) - oy, cx = (rc.yx >> 16) - ox;  // [0, TS)
                const int cell = cy * TS + cx;
                fr[k] = make_float2(rc.ly, rc.lx);
                key[k] = (cell << 16) | atomicAdd(&ccnt[cell], 1);
            }
        }
        __syncthreads();
        if (wave == 0) {  // exclusive scan of the 256 counts: 4 per lane + wave scan
            int v[4], s = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = ccnt[lane * 4 + i];
                s += v[i];
            }
            int incl = s;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int o = __shfl_up(incl, d, 64);
                if (lane >= d) incl += o;
            }
            int run = incl - s;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                cstart[lane * 4 + i] = run;
                run += v[i];
            }
            if (lane == 63) cstart[NCELL] = run;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < RPT; ++k) {
            if (key[k] < 0) continue;
            const int pos = cstart[key[k] >> 16] + (key[k] & 0xffff);
            sslot[pos] = (unsigned short)(tid + k * 512);
            sfrac[pos] = fr[k];
        }
        __syncthreads();

        // 2. pull every pixel of the window.  A wave takes PPW pixels at a time;
        //    lane (pixel slot ps, channel group co) sums the 16-byte slices (EPL
        //    channels) of all rows of its pixel's records, so one load instruction
        //    reads PPW whole rows.  Pixel (py, px) is corner 00 of cell (py, px),
        //    01 of (py, px-1), 10 of (py-1, px) and 11 of (py-1, px-1).
        //    Rows come in batches of 8 from buffer loads over the bucket's rows:
        //    a row index past the pixel's count reads 0 through an out-of-range
        //    offset, so no load sits in a branch, the compiler's load counting
        //    stays exact, and the next batch is in flight while one is summed
        //    (two register sets, the loop unrolled by two).
        typedef typename RowOf<T>::type R;   // element type of the rows
        constexpr int EPL = 16 / sizeof(T);  // channels per lane per row
        constexpr int LPR = KC / EPL;        // lanes per row (8)
        constexpr int PPW = 64 / LPR;        // pixels per wave pass (8)
        constexpr int NLD = EPL * sizeof(R) / 16;  // 16-byte loads per lane per row
        static_assert(LPR == 8, "a lane slice of a KC-channel row; 8-lane swizzle groups");
        typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
        const int co = lane % LPR, ps = lane / LPR;
        const int row_bytes = p.Cgp * (int)sizeof(R);
        // bf16 rows: this lane's 8 channels lie in 32-channel block co / 4 of the chunk
        const int sc_shift = 8 * (co >> 2);
        for (int cc = 0; cc < cpg; ++cc) {
            if constexpr (kRowScaled<T>) {
                // the chunk's scale codes of the batch's rows, in sorted order
                if (cc > 0) __syncthreads();  // the previous chunk is done with ssc
                const unsigned short *rsc16 =
                    reinterpret_cast<const unsigned short *>(p.rsc) + ((size_t)row0 + base) * cpg + cc;
                for (int i = tid; i < nrec; i += 512) ssc[i] = rsc16[(size_t)sslot[i] * cpg];
                __syncthreads();
            }
            // buffer over the batch's rows from this chunk's first channel (uniform);
            // the lane's slice goes into the offset
            const R *rows = (const R *)p.cgm + ((size_t)row0 + base) * p.Cgp + cc * KC;
            const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<R *>(rows), (short)0, nrec * row_bytes, 0x00020000);
            const int slice = co * 16 * NLD;
            // Passes of PPW pixels: pass qp < NSEG takes window row qp / 2,
            // columns 1 + 8 (qp % 2) .. +7 (8 of the tile's own pixels, 8-aligned
            // in the image); the later passes take the left ring column (px = 0)
            // PPW rows at a time.
            constexpr int NSEG = 2 * TW, NPASS = NSEG + (TW + PPW - 1) / PPW;
            static_assert(PPW == 8 && 1 + 8 * 2 == TW, "two 8-pixel segments per window row");
            for (int qp = wave; qp < NPASS; qp += 8) {
                const bool seg = qp < NSEG;  // (uniform over the wave)
                const int py = seg ? qp >> 1 : (qp - NSEG) * PPW + ps;
                const int px = seg ? 1 + 8 * (qp & 1) + ps : 0;
                const bool inwin = py < TW;
                const int Y = oy + py, X = ox + px;
                const bool live = inwin && Y >= 0 && Y < p.H && X >= 0 && X < p.W;
                // record ranges of the four cells whose corner q is this pixel
                int beg[4], len[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int cy = py - (q >> 1), cx = px - (q & 1);
                    const bool in = live && cy >= 0 && cy < TS && cx >= 0 && cx < TS;
                    const int cell = in ? cy * TS + cx : 0;
                    beg[q] = in ? cstart[cell] : 0;
                    len[q] = in ? cstart[cell + 1] - beg[q] : 0;
                }
                const int e1 = len[0], e2 = e1 + len[1], e3 = e2 + len[2], tot = e3 + len[3];
                float sum[EPL];
#pragma unroll
                for (int e = 0; e < EPL; ++e) sum[e] = 0.0f;
                // Row j of the pixel's corner-ordered record ranges: its record
                // position, weight and row offset (out of range past the pixel's
                // count), by selects only.  Lane co of the pixel's 8-lane group
                // works out row jb + co of a batch of LPR rows; the batch's loads
                // take each row's offset and weight from its lane (ds_swizzle in
                // bit mode: lane (l & 0x18) | u of every 32-lane half), so the
                // index arithmetic is done once per row instead of once per lane.
                auto row_info = [&](int jb, int &off, float &w, int &sc) __attribute__((always_inline)) {
                    const int j = jb + co;
                    const bool ok = j < tot, q1 = j >= e1, q2 = j >= e2, q3 = j >= e3;
                    int pos = beg[0] + j;
                    pos = q1 ? beg[1] + j - e1 : pos;
                    pos = q2 ? beg[2] + j - e2 : pos;
                    pos = q3 ? beg[3] + j - e3 : pos;
                    pos = ok ? pos : 0;
                    const float2 f = sfrac[pos];
                    const float wy = q2 ? f.x : 1.0f - f.x;             // corners 10, 11
                    const float wx = (q1 != q2) || q3 ? f.y : 1.0f - f.y;  // corners 01, 11
                    w = ok ? wy * wx : 0.0f;
                    off = ok ? (int)sslot[pos] * row_bytes : kGatherOutOfRange;
                    sc = kRowScaled<T> ? (int)ssc[kRowScaled<T> ? pos : 0] : 0;
                };
                auto fetch = [&](int off, float w, int sc, u32x4 (&raw)[LPR][NLD], float (&wgt)[LPR]) __attribute__((always_inline)) {
                    static_for<0, LPR>([&](auto uc) __attribute__((always_inline)) {
                        constexpr int u = decltype(uc)::value;
                        const int ou = __builtin_amdgcn_ds_swizzle(off, (u << 5) | 0x18);
                        wgt[u] = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(w), (u << 5) | 0x18));
                        if constexpr (kRowScaled<T>) {
                            const int scu = __builtin_amdgcn_ds_swizzle(sc, (u << 5) | 0x18);
                            wgt[u] *= row_unscale(((unsigned)scu >> sc_shift) & 0xffu);
                        }
                        // row_bytes is a multiple of 128 * NLD (the slice's range)
                        // and the marker has the low bits set, so OR-ing the slice
                        // in keeps either in range
#pragma unroll
                        for (int h = 0; h < NLD; ++h)
                            raw[u][h] = __builtin_amdgcn_raw_buffer_load_b128(rrs, ou | (slice + 16 * h), 0, 0);
                    });
                };
                auto accumulate = [&](const u32x4 (&raw)[LPR][NLD], const float (&wgt)[LPR]) __attribute__((always_inline)) {
                    constexpr int EU = 16 / sizeof(R);  // channels per 16-byte load
#pragma unroll
                    for (int u = 0; u < LPR; ++u) {
#pragma unroll
                        for (int h = 0; h < NLD; ++h) {
                            float v[EU];
                            Unpack<R>::run(make_uint4(raw[u][h].x, raw[u][h].y, raw[u][h].z, raw[u][h].w), v);
#pragma unroll
                            for (int e = 0; e < EU; ++e) sum[h * EU + e] = fmaf(wgt[u], v[e], sum[h * EU + e]);
                        }
                    }
                };
                u32x4 ra[LPR][NLD], rb[LPR][NLD];
                float wa[LPR], wb[LPR];
                int oa, ob, sa, sb;
                float xa, xb;
                // (scheduling barriers keep each batch's loads ahead of the sums of
                // the previous one; left alone the scheduler groups the fetches)
                row_info(0, oa, xa, sa);
                fetch(oa, xa, sa, ra, wa);
                for (int j0 = 0; j0 < tot; j0 += 2 * LPR) {
                    row_info(j0 + LPR, ob, xb, sb);
                    fetch(ob, xb, sb, rb, wb);
                    __builtin_amdgcn_sched_barrier(0);
                    accumulate(ra, wa);
                    __builtin_amdgcn_sched_barrier(0);
                    row_info(j0 + 2 * LPR, oa, xa, sa);
                    fetch(oa, xa, sa, ra, wa);
                    __builtin_amdgcn_sched_barrier(0);
                    accumulate(rb, wb);
                    __builtin_amdgcn_sched_barrier(0);
                }
                // Interior pixels (reachable from this tile's cells only) are this
                // block's alone.  With one batch their sums are final; with
                // several, the batches before the last keep the partial sums in
                // the bucket's gi_acc slot (the first writes them, so it needs
                // no clearing) and the last adds them back.  The accumulator's padding channels
                // (Cg..Cgp of a group) are never read back, so whole 16-byte
                // pieces are written.
                const bool inner = py >= 1 && py <= TS - 1 && px >= 1 && px <= TS - 1;
                if (inner) {
                    if (live && (first || last || tot > 0)) {
                        f32x4 *d4 =
                            reinterpret_cast<f32x4 *>(gi + ((py - 1) * (TS - 1) + px - 1) * p.Cgp + cc * KC + co * EPL);
#pragma unroll
                        for (int i = 0; i < EPL / 4; ++i) {
                            f32x4 v = f32x4{sum[4 * i], sum[4 * i + 1], sum[4 * i + 2], sum[4 * i + 3]};
                            if (!first) v += d4[i];
                            if (!last) d4[i] = v;
#pragma unroll
                            for (int k = 0; k < 4; ++k) sum[4 * i + k] = v[k];
                        }
                    }
                } else if (inwin) {
                    // border ring: written in full every call (zeros included),
                    // summed by ring_final_kernel, no atomics.  Later batches add
                    // to it; this lane wrote the same entry in every earlier batch.
                    f32x4 *r4 = reinterpret_cast<f32x4 *>(
                        p.ring + ((size_t)bucket * kRing + ring_index(py, px)) * p.Cgp + cc * KC + co * EPL);
#pragma unroll
                    for (int i = 0; i < EPL / 4; ++i) {
                        f32x4 v = f32x4{sum[4 * i], sum[4 * i + 1], sum[4 * i + 2], sum[4 * i + 3]};
                        if (!first) v += r4[i];
                        r4[i] = v;
#pragma unroll
                        for (int k = 0; k < 4; ++k) sum[4 * i + k] = v[k];
                    }
                }
                // After the last batch, the pass's 8 pixels of the tile's own
                // 16 x 16 block (window rows and columns 1 .. TS) go straight to
                // grad_input in the caller's type and layout: the interior ones
                // final, those on window row or column TS (tile boundary) partial,
                // to be overwritten by ring_final_kernel.
                if (last && seg && py >= 1) {
                    T *const gout = (T *)p.gi_out;
                    const int C = p.G * p.Cg, c0 = cc * KC + co * EPL;
                    if (p.gi_nhwc) {
                        // lane: its EPL channels of its pixel
                        if (live && c0 < p.Cg) {
                            T *dst = gout + (((size_t)b * p.H + Y) * p.W + X) * C + g * p.Cg + c0;
                            if (p.gi_vec && c0 + EPL <= p.Cg) {
                                *reinterpret_cast<uint4 *>(dst) = pack16<T>(sum);
                            } else {
#pragma unroll
                                for (int e = 0; e < EPL; ++e)
                                    if (c0 + e < p.Cg) dst[e] = from_f32<T>(sum[e]);
                            }
                        }
                    } else {
                        // transposed through this wave's LDS: lane l then holds
                        // KC/8 consecutive pixels (from LPX) of channel l % KC
                        *reinterpret_cast<uint4 *>(&stage[wave][ps * KC + co * EPL]) = pack16<T>(sum);
                        constexpr int PPL = KC / 8;  // pixels per lane: 16 bytes
                        const int cl = lane % KC, lpx = (lane / KC) * PPL;
                        T v[PPL];
#pragma unroll
                        for (int e = 0; e < PPL; ++e) v[e] = stage[wave][(lpx + e) * KC + cl];
                        const int X0 = ox + 1 + 8 * (qp & 1) + lpx, cgi = cc * KC + cl;
                        if (Y < p.H && X0 < p.W && cgi < p.Cg) {
                            T *dst = gout + (((size_t)b * C + g * p.Cg + cgi) * p.H + Y) * p.W + X0;
                            if (p.gi_vec && X0 + PPL <= p.W) {
                                *reinterpret_cast<uint4 *>(dst) = __builtin_bit_cast(uint4, v);
                            } else {
#pragma unroll
                                for (int e = 0; e < PPL; ++e)
                                    if (X0 + e < p.W) dst[e] = v[e];
                            }
                        }
                    }
                }
            }
        }
    }  // batches
}

// ---------------------------------------------------------------------------
// grad_input by cells (the default; dcn2_gi_gather_kernel is the per-pixel
// form).  One block per bucket (image, group, 16x16 cell tile).  For each
// chunk of KC channels, the window of (TS+1)^2 pixels the tile's corners can
// reach is accumulated in LDS in fp32, so every hand-off row is read once:
// the bucket's records are counting-sorted by cell (in batches of up to
// kGatherBatch; a bucket of one batch is sorted once for all its chunks), and
// a group of 8 lanes (lane = EPL-channel slice) takes one cell, sums its rows
// into the cell's four corner sums S_q = sum over the cell's records of
// (bilinear corner weight q) x (masked column-gradient row), and adds S_q to
// pixel (cy + q/2, cx + q%2) of the window by a plain read-add-write, with no
// atomics: wave w takes cell row 2w, then (after a barrier) 2w + 1, 8 cells
// at a time, so no two waves touch one window row at once, and within the
// wave the four corners are added one after another (a wave's LDS operations
// complete in order, so the neighbouring group's add to a shared pixel is
// seen).  Then the one-pixel border ring, shared with the neighbouring tiles,
// goes to the bucket's ring, every entry every call (zeros included), and the
// tile's 16 x 16 pixels straight to grad_input in the caller's type and layout;
// ring_final_kernel completes the tile-boundary pixels from the rings.  The
// reference scatters one global atomic per (sample, corner, channel)
// (com.cu:553-609).
// Mean samples per bucket from which the host takes dcn2_gi_push_kernel.
constexpr int kPushMinPerBucket = 1024;

template <typename T>
__global__ __launch_bounds__(512) void dcn2_gi_push_kernel(const BwdParams p) {
    constexpr int KC = Mma<T>::KC;  // channels per pass
    constexpr int TS = kCellTile, TW = TS + 1, NCELL = TS * TS;
    constexpr int RPT = kGatherBatch / 512;
    typedef typename RowOf<T>::type R;   // element type of the rows
    constexpr int EPL = 16 / sizeof(T);  // channels per lane
    constexpr int LPR = KC / EPL;        // lanes per row (8)
    constexpr int NLD = EPL * sizeof(R) / 16;  // 16-byte loads per lane per row
    constexpr int RPB = NLD == 1 ? 8 : 4;      // rows per batch of a lane group
    constexpr int EU = 16 / sizeof(R);         // channels per 16-byte load
    constexpr int NPC = EPL / 4;               // 16-byte window pieces per lane
    static_assert(LPR == 8 && RPB <= LPR && TS == 2 * 8, "8-lane groups; two cell rows per wave");
    __shared__ int ccnt[NCELL];
    __shared__ int cstart[NCELL + 1];
    __shared__ unsigned short sslot[kGatherBatch];  // row in the batch, sorted by cell
    __shared__ float2 sfrac[kGatherBatch];          // (ly, lx), sorted by cell
    __shared__ unsigned short ssc[kRowScaled<T> ? kGatherBatch : 1];  // bf16 rows: the chunk's scale codes
    // window [pixel][KC channels]: the lane's piece h (channels co*EPL + 4h ..)
    // at 16-byte slot h*LPR + co of its pixel, so the 8 lanes of a group
    // touch 8 consecutive slots per access
    __shared__ __attribute__((aligned(16))) float win[TW * TW * KC];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nb = p.B * p.G * p.nty * p.ntx;
    const int bucket = xcd_remap(blockIdx.x, nb);
    const int tx = bucket % p.ntx, ty = (bucket / p.ntx) % p.nty;
    const int bg = bucket / (p.ntx * p.nty), b = bg / p.G, g = bg - b * p.G;
    const int row0 = p.bstart[bucket], count = p.bstart[bucket + 1] - row0;
    const int oy = ty * TS - 1, ox = tx * TS - 1;  // pixel of local (0, 0)
    const int cpg = p.Cgp / KC;
    const int co = lane % LPR, gq = lane / LPR;
    const int row_bytes = p.Cgp * (int)sizeof(R);
    const int slice = co * 16 * NLD;
    // bf16 rows: this lane's 8 channels lie in 32-channel block co / 4 of the chunk
    const int sc_shift = 8 * (co >> 2);
    auto piece = [&](int pix, int h) __attribute__((always_inline)) {
        return reinterpret_cast<f32x4 *>(win + pix * KC) + h * LPR + co;
    };
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

    for (int cc = 0; cc < cpg; ++cc) {
        if (cc > 0) __syncthreads();  // the previous chunk's window is written out
        for (int i = tid; i < TW * TW * KC / 4; i += 512)
            reinterpret_cast<f32x4 *>(win)[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        for (int base = 0; base < count; base += kGatherBatch) {
            const int nrec = min(count - base, kGatherBatch);
            __syncthreads();  // the window is clear / the previous batch is done with the LDS arrays
            if (cc == 0 || count > kGatherBatch) {
                // 1. counting sort by cell (cell = local row * TS + local column)
                const BucketRec *__restrict__ recs = p.rec + (size_t)row0 + base;
                for (int i = tid; i < NCELL; i += 512) ccnt[i] = 0;
                __syncthreads();
                int key[RPT];  // (cell << 16) | rank, or -1
                float2 fr[RPT];
#pragma unroll
                for (int k = 0; k < RPT; ++k) {
                    const int r = tid + k * 512;
                    key[k] = -1;
                    fr[k] = make_float2(0.f, 0.f);
                    if (r < nrec) {
                        const BucketRec rc = recs[r];
                        const int cy = (int)(short)(rc.yx & 0xffff) - oy, cx = (rc.yx >> 16) - ox;  // [0, TS)
                        const int cell = cy * TS + cx;
                        fr[k] = make_float2(rc.ly, rc.lx);
                        key[k] = (cell << 16) | atomicAdd(&ccnt[cell], 1);
                    }
                }
                __syncthreads();
                if (wave == 0) {  // exclusive scan of the 256 counts: 4 per lane + wave scan
                    int v[4], sc = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        v[i] = ccnt[lane * 4 + i];
                        sc += v[i];
                    }
                    int incl = sc;
#pragma unroll
                    for (int d = 1; d < 64; d <<= 1) {
                        const int o = __shfl_up(incl, d, 64);
                        if (lane >= d) incl += o;
                    }
                    int run = incl - sc;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        cstart[lane * 4 + i] = run;
                        run += v[i];
                    }
                    if (lane == 63) cstart[NCELL] = run;
                }
                __syncthreads();
#pragma unroll
                for (int k = 0; k < RPT; ++k) {
                    if (key[k] < 0) continue;
                    const int pos = cstart[key[k] >> 16] + (key[k] & 0xffff);
                    sslot[pos] = (unsigned short)(tid + k * 512);
                    sfrac[pos] = fr[k];
                }
                __syncthreads();
            }
            if constexpr (kRowScaled<T>) {
                // the chunk's scale codes of the batch's rows, in sorted order
                // (the barrier at the batch's start ordered the last reads of ssc)
                const unsigned short *rsc16 =
                    reinterpret_cast<const unsigned short *>(p.rsc) + ((size_t)row0 + base) * cpg + cc;
                for (int i = tid; i < nrec; i += 512) ssc[i] = rsc16[(size_t)sslot[i] * cpg];
                __syncthreads();
            }

            // 2. the cells.  Rows come in batches of RPB per lane group from
            //    buffer loads over the batch's rows: a row index past the cell's
            //    count reads 0 through an out-of-range offset, so no load sits in
            //    a branch, and the next batch is in flight while one is summed
            //    (two register sets, the loop unrolled by two).  Lane co of the
            //    group works out row jb + co (co < RPB); the batch's loads take
            //    each row's offset and fractions from that lane (ds_swizzle in
            //    bit mode: lane (l & 0x18) | u of every 32-lane half).
            const R *rows = (const R *)p.cgm + ((size_t)row0 + base) * p.Cgp + cc * KC;
            const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<R *>(rows), (short)0, nrec * row_bytes, 0x00020000);
            // The group's four cells (round r: cell row 2 wave + r / 2, cells
            // 8 (r % 2) ..) form one stream of row batches: every round takes
            // the wave's largest cell in ceil(max / RPB) batches (at least one,
            // so every round reaches its window adds and round 1 its barrier),
            // and the batch after the one being summed is always in flight,
            // also across a round's window adds and the barrier (which waits
            // for LDS operations only).  So a wave's rounds do not each wait
            // for a round trip to memory.
            int rbeg[4], rtot[4], nbat[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int cell = (2 * wave + (r >> 1)) * TS + 8 * (r & 1) + gq;
                rbeg[r] = cstart[cell];
                rtot[r] = cstart[cell + 1] - rbeg[r];
                int tmax = rtot[r];
#pragma unroll
                for (int d = 8; d < 64; d <<= 1) tmax = max(tmax, __shfl_xor(tmax, d, 64));
                nbat[r] = max(1, (tmax + RPB - 1) / RPB);  // wave-uniform
            }
            const int nstream = nbat[0] + nbat[1] + nbat[2] + nbat[3];
            auto pick = [](const int (&a)[4], int r) __attribute__((always_inline)) {
                return r == 0 ? a[0] : (r == 1 ? a[1] : (r == 2 ? a[2] : a[3]));
            };
            // batch jb of round r: the row offset, fractions of row jb*RPB + co
            auto row_info = [&](int r, int jb, int &off, float &ly, float &lx, int &sc) __attribute__((always_inline)) {
                const int j = jb * RPB + co;
                const bool ok = co < RPB && j < pick(rtot, r);
                const int pos = ok ? pick(rbeg, r) + j : 0;
                const float2 f = sfrac[pos];
                ly = ok ? f.x : 0.0f;
                lx = ok ? f.y : 0.0f;
                off = ok ? (int)sslot[pos] * row_bytes : kGatherOutOfRange;
                sc = kRowScaled<T> ? (int)ssc[kRowScaled<T> ? pos : 0] : 0;
            };
            // A batch in flight: the RPB rows' loads (each lane's slice of
            // row u comes from lane u of its group) and this lane's own row's
            // fractions, handed out to the group when the batch is summed.
            struct Batch {
                u32x4 raw[RPB][NLD];
                float ly, lx;
                int sc;
            };
            auto fetch = [&](int off, float ly, float lx, int sc, Batch &bt) __attribute__((always_inline)) {
                bt.ly = ly;
                bt.lx = lx;
                bt.sc = sc;
                static_for<0, RPB>([&](auto uc) __attribute__((always_inline)) {
                    constexpr int u = decltype(uc)::value;
                    const int ou = __builtin_amdgcn_ds_swizzle(off, (u << 5) | 0x18);
                    // row_bytes is a multiple of 128 * NLD (the slice's range)
                    // and the marker has the low bits set, so OR-ing the slice
                    // in keeps either in range
#pragma unroll
                    for (int h = 0; h < NLD; ++h)
                        bt.raw[u][h] = __builtin_amdgcn_raw_buffer_load_b128(rrs, ou | (slice + 16 * h), 0, 0);
                });
            };
            float S[4][EPL];
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < EPL; ++e) S[q][e] = 0.0f;
            auto accumulate = [&](const Batch &bt) __attribute__((always_inline)) {
                static_for<0, RPB>([&](auto uc) __attribute__((always_inline)) {
                    constexpr int u = decltype(uc)::value;
                    float fy = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(bt.ly), (u << 5) | 0x18));
                    const float fx = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(bt.lx), (u << 5) | 0x18));
                    float hy = 1.0f - fy;
                    const float hx = 1.0f - fx;
                    if constexpr (kRowScaled<T>) {
                        // the inverse scale of the lane's 32-channel block of row u
                        const int scu = __builtin_amdgcn_ds_swizzle(bt.sc, (u << 5) | 0x18);
                        const float f = row_unscale(((unsigned)scu >> sc_shift) & 0xffu);
                        hy *= f;
                        fy *= f;
                    }
                    const float w[4] = {hy * hx, hy * fx, fy * hx, fy * fx};
#pragma unroll
                    for (int h = 0; h < NLD; ++h) {
                        float v[EU];
                        Unpack<R>::run(make_uint4(bt.raw[u][h].x, bt.raw[u][h].y, bt.raw[u][h].z, bt.raw[u][h].w), v);
#pragma unroll
                        for (int q = 0; q < 4; ++q)
#pragma unroll
                            for (int e = 0; e < EU; ++e) S[q][h * EU + e] = fmaf(w[q], v[e], S[q][h * EU + e]);
                    }
                });
            };
            // corner q of the group's cell of round r: pixel (cy + q/2, cx + q%2);
            // corner 01 of this group and corner 00 of the next group share a
            // pixel, so the corners go one after another (the compiler barrier
            // keeps each corner's reads after the previous corner's writes)
            auto window_add = [&](int r) __attribute__((always_inline)) {
                const int cy = 2 * wave + (r >> 1), cx = 8 * (r & 1) + gq;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int pix = (cy + (q >> 1)) * TW + cx + (q & 1);
                    f32x4 t[NPC];
#pragma unroll
                    for (int h = 0; h < NPC; ++h) t[h] = *piece(pix, h);
#pragma unroll
                    for (int h = 0; h < NPC; ++h) {
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            t[h][k] += S[q][4 * h + k];
                            S[q][4 * h + k] = 0.0f;
                        }
                        *piece(pix, h) = t[h];
                    }
                    asm volatile("" ::: "memory");
                }
            };
            // stream cursors (wave-uniform): fetch point (fr, fj), sum point (cr, cj)
            int fr = 0, fj = 0, cr = 0, cj = 0;
            auto fetch_next = [&](Batch &bt) __attribute__((always_inline)) {
                if (fr < 4) {
                    int off, sc;
                    float ly, lx;
                    row_info(fr, fj, off, ly, lx, sc);
                    fetch(off, ly, lx, sc, bt);
                    if (++fj == pick(nbat, fr)) {
                        ++fr;
                        fj = 0;
                    }
                }
            };
            // after summing batch (cr, cj): at a round's end, its window adds;
            // after round 1, the barrier between the even and the odd cell rows
            auto sum_done = [&]() __attribute__((always_inline)) {
                if (++cj == pick(nbat, cr)) {
                    window_add(cr);
                    if (cr == 1) __syncthreads();  // the even cell rows' window rows are done
                    ++cr;
                    cj = 0;
                }
            };
            // three batches rotate: while one is summed, the next two are in
            // flight (scheduling barriers keep each batch's loads ahead of the
            // sums of the previous one)
            Batch ba, bb, bc;
            fetch_next(ba);
            fetch_next(bb);
            for (int sidx = 0; sidx < nstream; sidx += 3) {
                fetch_next(bc);
                __builtin_amdgcn_sched_barrier(0);
                accumulate(ba);
                sum_done();
                __builtin_amdgcn_sched_barrier(0);
                if (sidx + 1 >= nstream) break;
                fetch_next(ba);
                __builtin_amdgcn_sched_barrier(0);
                accumulate(bb);
                sum_done();
                __builtin_amdgcn_sched_barrier(0);
                if (sidx + 2 >= nstream) break;
                fetch_next(bb);
                __builtin_amdgcn_sched_barrier(0);
                accumulate(bc);
                sum_done();
                __builtin_amdgcn_sched_barrier(0);
            }
        }  // batches
        __syncthreads();

        // 3. the window: the border ring to the bucket's ring (for
        //    ring_final_kernel); then the tile's pixels (16ty .. +15, 16tx ..
        //    +15) = window (1 .. TS, 1 .. TS) straight to grad_input in the
        //    caller's type and layout.  Of those, the pixels on row or column TS
        //    are partial sums here; ring_final_kernel, launched after this
        //    kernel, overwrites every such (tile-boundary) pixel with the full
        //    sum.
        {
            for (int pl = 8 * wave + gq; pl < TW * TW; pl += 64) {
                const int py = pl / TW, px = pl - py * TW;
                if (py >= 1 && py <= TS - 1 && px >= 1 && px <= TS - 1) continue;
                f32x4 *d4 = reinterpret_cast<f32x4 *>(
                    p.ring + ((size_t)bucket * kRing + ring_index(py, px)) * p.Cgp + cc * KC + co * EPL);
#pragma unroll
                for (int h = 0; h < NPC; ++h) d4[h] = *piece(pl, h);
            }
            // window value of channel cl (of this chunk) at pixel slot pix: cl =
            // co * EPL + 4h + k lives at 16-byte slot h * LPR + co, element k
            auto win_at = [&](int pix, int cl) __attribute__((always_inline)) {
                const int c_o = cl / EPL, rem = cl - c_o * EPL;
                return win[pix * KC + ((rem >> 2) * LPR + c_o) * 4 + (rem & 3)];
            };
            T *const gout = (T *)p.gi_out;
            const int C = p.G * p.Cg;
            if (p.gi_nhwc) {
                // item: pixel (yy, xx) of the tile, 8 channels 8j ..
                constexpr int NPP = KC / 8;
                for (int it = tid; it < TS * TS * NPP; it += 512) {
                    const int j = it % NPP, pl = it / NPP;
                    const int yy = pl / TS, xx = pl - yy * TS;
                    const int Y = ty * TS + yy, X = tx * TS + xx, c0 = cc * KC + 8 * j;
                    if (Y >= p.H || X >= p.W || c0 >= p.Cg) continue;
                    const int pix = (yy + 1) * TW + xx + 1;
                    T v[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = from_f32<T>(win_at(pix, 8 * j + e));
                    T *dst = gout + (((size_t)b * p.H + Y) * p.W + X) * C + g * p.Cg + c0;
                    if (p.gi_vec && c0 + 8 <= p.Cg) {
                        store8(dst, v);
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            if (c0 + e < p.Cg) dst[e] = v[e];
                    }
                }
            } else {
                // item: channel cl (consecutive lanes: consecutive channels),
                // row yy of the tile, pixels 8hx .. 8hx + 7
                for (int it = tid; it < KC * TS * 2; it += 512) {
                    const int cl = it % KC, r2 = it / KC;
                    const int yy = r2 >> 1, hx = r2 & 1;
                    const int Y = ty * TS + yy, X0 = tx * TS + 8 * hx, cg = cc * KC + cl;
                    if (Y >= p.H || X0 >= p.W || cg >= p.Cg) continue;
                    const int pix = (yy + 1) * TW + 8 * hx + 1;
                    T v[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = from_f32<T>(win_at(pix + e, cl));
                    T *dst = gout + (((size_t)b * C + g * p.Cg + cg) * p.H + Y) * p.W + X0;
                    if (p.gi_vec && X0 + 8 <= p.W) {
                        store8(dst, v);
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            if (X0 + e < p.W) dst[e] = v[e];
                    }
                }
            }
            // (the chunk loop's barrier orders these reads before the next clear)
        }
    }  // channel chunks
}

// gw_acc [Mp][Kp] (K order tap, group, channel) -> grad_weight [Cout][C][kh][kw];
// gb_acc -> grad_bias.  nblk workgroups of 256 threads; ring_final_kernel runs
// them as extra workgroups of its own launch (finalize_gw_kernel alone for an
// empty batch).
template <typename T> struct GwFinal {
    const float *gwa, *gba;
    T *gw, *gb;
    int Cout, Cw, mpg, KK, Cg, Cgp, G, Kp;
    long nblk;
};
template <typename T>
__device__ __forceinline__ void finalize_gw_block(const GwFinal<T> &f, long blk) {
    // grad_weight [Cout][Cw][KK]: row m's channel cl is input channel
    // (m / mpg) * Cw + cl, the diagonal block of the block-diagonal W'.
    // (32-bit index math: the host bounds Mp * Kp, and so Cout * Cw * KK,
    // below 2^31)
    const int idx = (int)blk * 256 + (int)threadIdx.x;
    const int total = f.Cout * f.Cw * f.KK;
    if (idx < total) {
        const int m = idx / (f.Cw * f.KK);
        const int r = idx - m * f.Cw * f.KK;
        const int cl = r / f.KK, tap = r - cl * f.KK;
        const int c = (m / f.mpg) * f.Cw + cl;
        const int g = c / f.Cg, ci = c - g * f.Cg;
        f.gw[idx] = (T)f.gwa[(size_t)m * f.Kp + ((size_t)tap * f.G + g) * f.Cgp + ci];
    }
    if (f.gb && idx < f.Cout) f.gb[idx] = (T)f.gba[idx];
}
template <typename T>
__global__ __launch_bounds__(256) void finalize_gw_kernel(const GwFinal<T> f) {
    finalize_gw_block(f, blockIdx.x);
}

// The tile-boundary pixels of a directly written grad_input (see
// dcn2_gi_push_kernel with gi_out): the sums of the border rings that hold
// each pixel, written in the caller's type and layout over the per-tile
// partial value the per-cell kernel left there.  Pixel (Y, X) is a boundary
// pixel when Y % TS == TS-1 (a boundary row) or X % TS == TS-1 (a boundary
// column); it is (py, px) = ((Y+1) % TS, (X+1) % TS) of the window of tile
// ((Y+1) / TS, (X+1) / TS), and also row TS of the tile above when py == 0
// and column TS of the tile to the left when px == 0.  One launch, 256
// threads per block, four block ranges:
//   [0, nb_rows)  NCHW boundary rows: 64 pixels x 32 padded channels per
//                 block, ring sums -> LDS -> 16-byte stores of 8 pixels of
//                 one channel (stores along pixels, as the rows are
//                 contiguous in NCHW);
//   then          the other boundary pixels (all of them for channels-last),
//                 one thread per pixel and 4 padded channels;
//   then          grad_offset / grad_mask of the fused kernel's groups of
//                 several chunks (corner_finish), one thread per sample;
//   then          grad_weight / grad_bias (their accumulators are complete
//                 when this kernel runs).
struct RingFinal {
    int nrow, ncol;       // boundary rows and columns of an image
    int xblk, cblk;       // NCHW row part: 64-pixel blocks per row, 32-channel blocks
    long nb_rows;         // blocks of the NCHW row part
    long items;           // items of the per-thread part
    long nb_items;        // its blocks
    long nb_corner;       // blocks of the fused kernel's corner-sum finish (0: none)
};
__device__ __forceinline__ f32x4 ring_sum(const BwdParams &p, int b, int g, int ci, int Y, int X) {
    constexpr int TS = kCellTile;
    const int py = (Y + 1) % TS, ty = (Y + 1) / TS, px = (X + 1) % TS, tx = (X + 1) / TS;
    f32x4 v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if (i == 1 && (py != 0 || ty == 0)) continue;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            if (jj == 1 && (px != 0 || tx == 0)) continue;
            const long bucket = (((long)b * p.G + g) * p.nty + (ty - i)) * p.ntx + (tx - jj);
            v += *reinterpret_cast<const f32x4 *>(
                p.ring + (bucket * kRing + ring_index(i ? TS : py, jj ? TS : px)) * p.Cgp + ci);
        }
    }
    return v;
}
template <typename T>
__global__ __launch_bounds__(256) void ring_final_kernel(const BwdParams p, const RingFinal r,
                                                         const GwFinal<T> f) {
    constexpr int TS = kCellTile;
    const int H = p.H, W = p.W, Cgp = p.Cgp, cs = p.G * p.Cgp, q4 = cs / 4;
    const int C = p.G * p.Cg;
    T *const gout = (T *)p.gi_out;
    const long blk = blockIdx.x;
    if (blk < r.nb_rows) {
        __shared__ float tile[64][33];
        const int xb = (int)(blk % r.xblk);
        long rest = blk / r.xblk;
        const int cb = (int)(rest % r.cblk);
        rest /= r.cblk;
        const int k = (int)(rest % r.nrow), b = (int)(rest / r.nrow);
        const int Y = TS * k + TS - 1, X0 = xb * 64, cp0 = cb * 32;
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int pl = (tid >> 3) + 32 * i, c4 = (tid & 7) * 4;
            const int X = X0 + pl, cp = cp0 + c4, g = cp / Cgp, ci = cp - g * Cgp;
            const f32x4 v = X < W ? ring_sum(p, b, g, ci, Y, X) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int e = 0; e < 4; ++e) tile[pl][c4 + e] = v[e];
        }
        __syncthreads();
        const int cl = tid >> 3, p8 = (tid & 7) * 8;
        const int cp = cp0 + cl, g = cp / Cgp, ci = cp - g * Cgp;
        const int X = X0 + p8;
        if (ci >= p.Cg || X >= W) return;
        T v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = from_f32<T>(tile[p8 + e][cl]);
        T *dst = gout + (((size_t)b * C + g * p.Cg + ci) * H + Y) * W + X;
        if (p.gi_vec && X + 8 <= W) {
            store8(dst, v);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (X + e < W) dst[e] = v[e];
        }
        return;
    }
    if (blk < r.nb_rows + r.nb_items) {
        const long item = (blk - r.nb_rows) * 256 + threadIdx.x;
        if (item >= r.items) return;
        // pixels: (NHWC only) the boundary rows, then the boundary columns
        // outside the boundary rows, image by image
        const long k0 = item / q4;
        const int cp = (int)(item - k0 * q4) * 4;
        const long rows_px = p.gi_nhwc ? (long)r.nrow * W : 0;
        const long per_img = rows_px + (long)(H - r.nrow) * r.ncol;
        const int b = (int)(k0 / per_img);
        const long k = k0 - (long)b * per_img;
        int Y, X;
        if (k < rows_px) {
            Y = TS * (int)(k / W) + TS - 1;
            X = (int)(k % W);
        } else {
            const long k2 = k - rows_px;
            const int c = (int)(k2 / (H - r.nrow)), j = (int)(k2 % (H - r.nrow));
            Y = j + j / (TS - 1);  // the j-th row that is not a boundary row
            X = TS * c + TS - 1;
        }
        const int g = cp / Cgp, ci = cp - g * Cgp;
        if (ci >= p.Cg) return;  // padding channels only
        const f32x4 v = ring_sum(p, b, g, ci, Y, X);
        if (p.gi_nhwc) {
            T *dst = gout + (((size_t)b * H + Y) * W + X) * C + g * p.Cg + ci;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (ci + e < p.Cg) dst[e] = from_f32<T>(v[e]);
        } else {
            T *dst = gout + (((size_t)b * C + g * p.Cg + ci) * H + Y) * W + X;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (ci + e < p.Cg) dst[(size_t)e * H * W] = from_f32<T>(v[e]);
        }
        return;
    }
    const long cb = blk - r.nb_rows - r.nb_items;
    if (cb < r.nb_corner) {
        // grad_offset / grad_mask of groups of several chunks (csum is complete:
        // the fused kernel ran before the grad_input kernels)
        const int N = p.Ho * p.Wo, planes = p.G * p.kh * p.kw;
        const long sidx = cb * 256 + threadIdx.x;
        if (sidx < (long)p.B * planes * N) {
            const int n = (int)(sidx % N);
            const long bp = sidx / N;
            corner_finish<T>(p, n, (int)(bp % planes), (int)(bp / planes));
        }
        return;
    }
    const long gb = cb - r.nb_corner;
    if (gb < f.nblk) finalize_gw_block(f, gb);
}

// ---------------------------------------------------------------------------
// The fused kernel (column gradient and grad_weight in one pass) serves
// 2-byte types with Mp of 128 or 256 (one M chunk), and images of gO and xt
// below 2 GiB each; the launch also needs gO rows that take 16-byte loads.
// Groups of several K chunks (Cgp > KC) add their corner sums up in csum.
// Option DCN2_OPT_BWD_FUSED = 0 selects the two-kernel path for every shape
// (the tests compare both paths).
bool fused_bwd_shape(const Geo &g) {
    return g.esz == 2 && g.opt_fused != 0 && (g.Mp == 256 || g.Mp == 128) &&
           (long long)g.Cout * g.N * g.esz <= kGoOutOfRange &&
           (long long)g.H * g.W * g.cs * g.esz <= kGoOutOfRange;
}

template <typename T>
static hipError_t backward_t(const Geo &g, const BwdParams &p0, void *grad_input,
                             void *grad_weight, void *grad_bias, bool last, hipStream_t s) {
    BwdParams p = p0;
    hipError_t e;
    // (the fp32 grad_weight / grad_bias accumulators and the bucket counts
    // were zeroed by the pack launch; gi_acc, the per-pixel gather's partial
    // sums between the batches of a bucket, needs no clearing: the first batch
    // writes them)
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        ncu <= 0)
        ncu = 256;
    // grad_weight / grad_bias finalisation (run by the grad_input finalisation
    // launch of the last slice, or alone for an empty batch; the earlier
    // slices only accumulate, nblk = 0)
    GwFinal<T> gwf;
    gwf.gwa = p.gw_acc;
    gwf.gba = p.gb_acc;
    gwf.gw = (T *)grad_weight;
    gwf.gb = (T *)grad_bias;
    gwf.Cout = g.Cout;
    gwf.Cw = g.Cw;
    gwf.mpg = g.Cout / g.WG;
    gwf.KK = g.KK;
    gwf.Cg = g.Cg;
    gwf.Cgp = g.Cgp;
    gwf.G = g.G;
    gwf.Kp = g.Kp;
    gwf.nblk = last ? (std::max<long>((long)g.Cout * g.Cw * g.KK, g.Cout) + 255) / 256 : 0;
    const bool fused = fused_bwd_shape(g) && p.go_vec;
    long corner_blocks = 0;  // ring_final_kernel's corner-sum finish blocks
    if (g.B > 0) {
        // 2. column gradient: grad_offset, grad_mask, grad_input accumulation
        //    (and grad_weight / grad_bias when fused)
        prof_begin(DCN2_STAGE_BWD_BUCKET, s);
        {
            // buckets: count, scan, place (exact sizes, see dcn2_bucket_kernel)
            const int f32 = sizeof(T) == 4, isbf = std::is_same<T, bf16>::value;
            const int nbuckets = g.B * g.G * p.nty * p.ntx;
            const bool tab = (long)p.nty * p.ntx <= kBucketTab;
            const int fold = tab && nbuckets <= kBucketFold;  // bcnt, bstart, bcur cleared by the pack launch
            const dim3 bgrid(ceil_div(g.N, tab ? 256 * kBucketSPT : 256), g.G * g.KK, g.B);
            const size_t tab_bytes = (size_t)p.nty * p.ntx * sizeof(int);
            if (tab) dcn2_bucket_kernel<false><<<bgrid, 256, tab_bytes, s>>>(p, p.offset, f32, isbf, 0);
            else dcn2_bucket_global_kernel<false><<<bgrid, 256, 0, s>>>(p, p.offset, f32, isbf);
            if ((e = hipGetLastError()) != hipSuccess) return e;
            if (!fold) {
                dcn2_bucket_scan_kernel<<<1, 1024, 0, s>>>(p.bcnt, p.bstart, p.bcur, nbuckets);
                if ((e = hipGetLastError()) != hipSuccess) return e;
            }
            if (tab)
                dcn2_bucket_kernel<true><<<bgrid, 256, 2 * tab_bytes + sizeof(int), s>>>(p, p.offset, f32, isbf,
                                                                                        fold);
            else dcn2_bucket_global_kernel<true><<<bgrid, 256, 0, s>>>(p, p.offset, f32, isbf);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        prof_end(DCN2_STAGE_BWD_BUCKET, s);
        prof_begin(DCN2_STAGE_BWD_COLGRAD, s);
        {
            if constexpr (sizeof(T) == 2) {
                if (fused) {
                    // one workgroup per CU: each K chunk gets CUs/nch ranges of
                    // 64-pixel tiles
                    BwdParams pf = p;
                    const int cpg = g.Cgp / g.KC, nch = g.KK * g.G * cpg;
                    pf.tiles_per_img = ceil_div(g.N, 64);
                    pf.splits = std::max(1, std::min(ncu / nch, g.B * pf.tiles_per_img));
                    const int grid = pf.splits * nch;
#define DCN2_FUSED(MPV)                                                                     \
    do {                                                                                    \
        if (p.go_nhwc) dcn2_bwd_fused_kernel<T, true, MPV><<<grid, 512, 0, s>>>(pf);       \
        else dcn2_bwd_fused_kernel<T, false, MPV><<<grid, 512, 0, s>>>(pf);                \
    } while (0)
                    if (g.Mp == 256) DCN2_FUSED(256);
                    else DCN2_FUSED(128);
#undef DCN2_FUSED
                    if ((e = hipGetLastError()) != hipSuccess) return e;
                    // groups of several chunks: grad_offset / grad_mask from
                    // the corner sums the chunks added up in csum, finished by
                    // ring_final_kernel
                    corner_blocks = cpg > 1 ? ((long)g.B * g.G * g.KK * g.N + 255) / 256 : 0;
                }
            }
        }
        if (!fused) {
            dim3 grid(p.tiles_per_img, g.B);
            // W'^T staged in LDS when a chunk of it fits (Mp <= 256); gO resident
            // in registers when one M chunk covers all rows.  fp32 keeps the
            // 128-wide M chunk: 256 would hold 128 gO registers.
            const bool alds = g.Mp <= 256;
#define DCN2_COLGRAD(MCHV)                                                                      \
    do {                                                                                        \
        if (g.Mp == MCHV) dcn2_colgrad_kernel<T, MCHV, true, true><<<grid, 512, 0, s>>>(p);     \
        else if (alds) dcn2_colgrad_kernel<T, MCHV, true, false><<<grid, 512, 0, s>>>(p);       \
        else dcn2_colgrad_kernel<T, MCHV, false, false><<<grid, 512, 0, s>>>(p);                \
    } while (0)
            if constexpr (sizeof(T) == 2) {
                if (g.Mp % 256 == 0) DCN2_COLGRAD(256);
                else DCN2_COLGRAD(128);
            } else {
                DCN2_COLGRAD(128);
            }
#undef DCN2_COLGRAD
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        prof_end(DCN2_STAGE_BWD_COLGRAD, s);
        // 3. grad_weight / grad_bias of the two-kernel path
        auto run_gradw = [&]() -> hipError_t {
            prof_begin(DCN2_STAGE_BWD_GRADW, s);
            // weight groups split per group (Geo::gsplit): an M chunk must lie
            // in one group, whose rows are a multiple of 128
            const int cog = g.gsplit ? g.Cout / g.WG : 0;
            const int mb = (cog ? cog % 256 == 0 : g.Mp % 256 == 0) ? 8 : 4;
            p.gw_cpt = g.cpt;
            p.gw_cpw = g.cpw;
            p.gw_cog = cog;
            p.gw_nch = cog ? g.KK * g.cpw : g.Kp / g.KC;
            const int nch = p.gw_nch;
            const int nmc = g.Mp / (32 * mb);
            const int T_total = g.B * p.tiles_per_img;
            // One workgroup per CU: each (K chunk, M chunk) pair gets CUs/(nch*nmc)
            // contiguous pixel-tile ranges, so the partial grad_weight tiles a
            // workgroup adds with fp32 atomics are few (one set per range).
            int S = ncu / (nch * nmc);
            S = std::max(1, std::min(S, T_total));
            p.splits = S;
            const int grid = S * nch * nmc;
            bool line = false;  // 2-byte type with 16-byte gO rows: whole-line loads
#define DCN2_GRADW(KERN, ...) KERN<T, __VA_ARGS__><<<grid, 512, 0, s>>>(p)
#define DCN2_GRADW_MB(KERN, ...)                                                                 \
    do {                                                                                         \
        if (mb == 8) { if (p.mask) DCN2_GRADW(KERN, 8, true __VA_ARGS__);                        \
                       else DCN2_GRADW(KERN, 8, false __VA_ARGS__); }                            \
        else { if (p.mask) DCN2_GRADW(KERN, 4, true __VA_ARGS__);                                \
               else DCN2_GRADW(KERN, 4, false __VA_ARGS__); }                                    \
    } while (0)
            if constexpr (sizeof(T) == 2) {
                if (p.go_vec && (long long)g.Cout * g.N * (long long)sizeof(T) <= kGoOutOfRange) {
                    if (p.go_nhwc) DCN2_GRADW_MB(dcn2_gradw_line_kernel, , true);
                    else DCN2_GRADW_MB(dcn2_gradw_line_kernel, , false);
                    line = true;
                }
            }
            if (!line) DCN2_GRADW_MB(dcn2_gradw_kernel);
#undef DCN2_GRADW_MB
#undef DCN2_GRADW
            const hipError_t ge = hipGetLastError();
            prof_end(DCN2_STAGE_BWD_GRADW, s);
            return ge;
        };
        const GatherGeo gg = gather_geometry(g);
        const int nbk = (int)gg.nbuckets;
        const int nrow = g.H / kCellTile, ncol = g.W / kCellTile;
        // grad_weight first (when not fused), so that its finalisation can
        // ride in the last launch, ring_final_kernel, and before the border
        // rings overwrite xt (they may share its bytes, see bwd_workspace)
        if (!fused && (e = run_gradw()) != hipSuccess) return e;
        prof_begin(DCN2_STAGE_BWD_GATHER, s);
        // both grad_input kernels write the caller's grad_input directly (the
        // tile-boundary pixels partially; ring_final_kernel completes them)
        p.gi_out = grad_input;
        p.gi_nhwc = g.nhwc;
        const int align16 = ((uintptr_t)grad_input & 15) == 0;
        p.gi_vec = align16 && (g.nhwc ? g.C % 8 == 0 && g.Cg % 8 == 0 : g.W % 8 == 0);
        if (gg.by_cells) {
            dcn2_gi_push_kernel<T><<<nbk, 512, 0, s>>>(p);
        } else {
            // At most two workgroups per CU (extra LDS reserved at launch when
            // the static LDS leaves room for three): each bucket's rows are read
            // once per corner, and with three buckets per CU the rows in use no
            // longer fit an XCD's L2 (measured at c2: 138 us at three per CU,
            // 113 us at two, 119 us at one).
            int lds_cu = 0;
            if (hipDeviceGetAttribute(&lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor,
                                      dev) != hipSuccess)
                lds_cu = 0;
            const int pad = std::max(0, lds_cu / 3 + 256 - gather_static_lds(kRowScaled<T>));
            dcn2_gi_gather_kernel<T><<<nbk, 512, pad, s>>>(p);
        }
        if ((e = hipGetLastError()) != hipSuccess) return e;
        // the tile-boundary pixels from the border rings, and grad_weight /
        // grad_bias (see ring_final_kernel)
        RingFinal rf;
        rf.nrow = nrow;
        rf.ncol = ncol;
        rf.xblk = ceil_div(g.W, 64);
        rf.cblk = g.cs / 32;
        rf.nb_rows = g.nhwc ? 0 : (long)g.B * nrow * rf.xblk * rf.cblk;
        rf.items = (long)g.B * ((g.nhwc ? (long)nrow * g.W : 0) + (long)(g.H - nrow) * ncol) *
                   (g.cs / 4);
        rf.nb_items = (rf.items + 255) / 256;
        rf.nb_corner = corner_blocks;
        // (none in a slice before the last when the images have no
        // tile-boundary pixels and no corner sums to finish)
        const long rblocks = rf.nb_rows + rf.nb_items + rf.nb_corner + gwf.nblk;
        if (rblocks > 0) ring_final_kernel<T><<<(unsigned)rblocks, 256, 0, s>>>(p, rf, gwf);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        prof_end(DCN2_STAGE_BWD_GATHER, s);
    } else {
        // 5. (empty batch) grad_weight / grad_bias alone
        prof_begin(DCN2_STAGE_BWD_FINAL, s);
        finalize_gw_kernel<T><<<(unsigned)gwf.nblk, 256, 0, s>>>(gwf);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        prof_end(DCN2_STAGE_BWD_FINAL, s);
    }
    return hipSuccess;
}

GatherGeo gather_geometry(const Geo &g) {
    GatherGeo gg;
    gg.ntx = ceil_div(g.W + 1, kCellTile);
    gg.nty = ceil_div(g.H + 1, kCellTile);
    gg.nbuckets = (long)g.B * g.G * gg.ntx * gg.nty;
    // every sample is placed in at most one bucket
    gg.rows = (long)g.B * g.G * g.KK * g.N;
    gg.row_esz = row_elem_bytes(g.dtype);
    gg.row_scaled = row_scaled(g.dtype) ? 1 : 0;
    gg.batch_bytes = (long)kGatherBatch * g.Cgp * gg.row_esz;
    gg.max_batch_bytes = kGatherOutOfRange;
    // By cells (each row read once, one block per CU) when the buckets are
    // full enough to amortise a block's fixed work; per pixel otherwise.
    // Option DCN2_OPT_GI_PUSH = 1 / 0 forces either.  Measured: c2 68
    // against 72 us, c3 ~190 against 282 us (2304 samples per bucket); c4
    // (576 per bucket) ~118 against 73 us.
    gg.by_cells = g.opt_push >= 0 ? g.opt_push != 0
                                  : gg.rows >= (long)kPushMinPerBucket * gg.nbuckets;
    gg.acc_bytes = gg.rows / (kGatherBatch + 1) * (long)(kCellTile - 1) * (kCellTile - 1) * g.Cgp *
                   (long)sizeof(float);
    return gg;
}

hipError_t launch_backward(const Geo &g, const void *xt, const void *wt, const void *tab,
                           const void *offset,
                           const void *mask, const void *grad_out, void *grad_input,
                           void *grad_offset, void *grad_mask, void *grad_weight, void *grad_bias,
                           float *gi_acc, float *gw_acc, float *gb_acc, void *cgm, void *rsc,
                           float *csum, void *rec, int *bcnt, int *bstart, int *bcur, int *sidx,
                           float *ring, bool last, hipStream_t s) {
    BwdParams p;
    p.xt = xt;
    p.wt = wt;
    p.tab = tab;
    p.offset = offset;
    p.mask = mask;
    p.gout = grad_out;
    p.goff = grad_offset;
    p.gmask = grad_mask;
    p.off_bs = g.off_bs;
    p.msk_bs = g.msk_bs;
    p.msk_logit = mask ? g.msk_logit : 0;
    p.gi_acc = gi_acc;
    p.gw_acc = gw_acc;
    p.gb_acc = grad_bias ? gb_acc : nullptr;
    p.B = g.B;
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
    p.Cg = g.Cg;
    p.Cgp = g.Cgp;
    p.Ho = g.Ho;
    p.Wo = g.Wo;
    p.Kp = g.Kp;
    p.Mp = g.Mp;
    p.tiles_per_img = ceil_div(g.N, 128);
    p.splits = 1;
    p.go_nhwc = g.out_nhwc;
    p.go_vec = (g.out_nhwc ? g.Cout % 8 == 0 : g.N % 8 == 0) && (((uintptr_t)grad_out & 15) == 0);
    const GatherGeo gg = gather_geometry(g);
    p.cgm = cgm;
    p.rsc = (unsigned char *)rsc;
    p.csum = csum;
    p.rec = (BucketRec *)rec;
    p.bcnt = bcnt;
    p.bstart = bstart;
    p.bcur = bcur;
    p.sidx = sidx;
    p.ntx = gg.ntx;
    p.nty = gg.nty;
    p.ring = ring;
    p.gi_out = nullptr;  // (set by the by-cells grad_input)
    p.gi_nhwc = p.gi_vec = 0;
    switch (g.dtype) {
    case DCN2_F16: return backward_t<f16>(g, p, grad_input, grad_weight, grad_bias, last, s);
    case DCN2_BF16: return backward_t<bf16>(g, p, grad_input, grad_weight, grad_bias, last, s);
    default: return backward_t<float>(g, p, grad_input, grad_weight, grad_bias, last, s);
    }
}

}  // namespace dcn2
