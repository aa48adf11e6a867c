// Shared device-side definitions for the gfx950 DCNv2 kernels.
//
// Data layout in HBM (all workspace buffers are produced by dcn2_pack.hip):
//   xt  : input repacked channels-last, [B][H*W][G*Cgp] in the call dtype, where
//         Cgp = Cg rounded up to the channel chunk KC and the padding channels
//         are zero.  One bilinear corner of one pixel is then a contiguous
//         channel vector, fetched with 16-byte loads.
//   wp  : weight repacked [Mp][Kp] with K ordered (tap, group, channel):
//         k = (tap*G + g)*Cgp + c, rows padded to the block tile with zeros.
//         Row-contiguous K is the MFMA A-operand order for the forward.
//   wt  : the transpose [Kp][Mp] of wp (backward column-gradient GEMM).
// The GEMM is D[m][n] = sum_k wp[m][k] * col[k][n] where col is never written
// to HBM: a chunk of KC channels of one (tap, group) is sampled into LDS and
// consumed by MFMA directly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dcn2 {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// MFMA selection per element type.  All use the 32x32 output block whose
// accumulator layout is: acc[r] of lane l holds D[8*(r/4) + 4*(l/32) + r%4][l%32].
// A operand: lane l holds A[l%32][kq*KPL .. kq*KPL+KPL-1] with kq = l/32.
// B operand: lane l holds B[kq*KPL .. +KPL-1][l%32].
template <typename T> struct Mma;

template <> struct Mma<f16> {
    static constexpr int KPL = 8;     // K elements per lane per instruction
    static constexpr int KSTEP = 16;  // K per instruction
    static constexpr int KC = 64;     // channel chunk sampled per LDS stage
    typedef f16x8 frag;
    static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

template <> struct Mma<bf16> {
    static constexpr int KPL = 8;
    static constexpr int KSTEP = 16;
    static constexpr int KC = 64;
    typedef bf16x8 frag;
    static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

template <> struct Mma<float> {
    static constexpr int KPL = 1;
    static constexpr int KSTEP = 2;
    static constexpr int KC = 32;
    typedef float frag;
    static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
};

template <typename T> __device__ __forceinline__ float to_f32(T v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f32(float v) { return (T)v; }

// Modulation mask value from its stored value: the value itself, or
// sigmoid(v) when the mask buffer holds the predictor's logits (the
// reference's DCN module applies torch.sigmoid, dcn_v2_mm.py:137).
__device__ __forceinline__ float mask_value(float v, int logit) {
    return logit ? 1.0f / (1.0f + __expf(-v)) : v;
}

// Bilinear sampling descriptor of one (pixel, tap, group): the four corner
// element offsets inside one image of xt (0 for a corner outside the image)
// and the four corner weights with the modulation mask folded in (0 for a
// corner outside the image).  Matches reference com.cu:119-148 + 187: a
// corner outside [0,H-1]x[0,W-1] contributes nothing, so a sample outside
// (-1,H)x(-1,W) reads 0.
struct Corners {
    int off[4];   // (y0,x0) (y0,x1) (y1,x0) (y1,x1)
    float w[4];
};

// Sample position and validity for one (pixel, tap); also returns the
// fractional parts needed by the backward.  `y`, `x` are clamped to
// [-2, H+1] x [-2, W+1] first: every point outside (-1,H)x(-1,W) samples 0
// either way, and the clamp keeps the float->int conversion defined for
// arbitrarily large learned offsets.
struct SamplePos {
    int y0, x0;
    float ly, lx;
    bool vy0, vy1, vx0, vx1;
};

__device__ __forceinline__ SamplePos sample_pos(float y, float x, int H, int W) {
    SamplePos s;
    y = fminf(fmaxf(y, -2.0f), (float)H + 1.0f);
    x = fminf(fmaxf(x, -2.0f), (float)W + 1.0f);
    const float fy = floorf(y), fx = floorf(x);
    s.y0 = (int)fy;
    s.x0 = (int)fx;
    s.ly = y - fy;
    s.lx = x - fx;
    s.vy0 = (unsigned)s.y0 < (unsigned)H;
    s.vy1 = (unsigned)(s.y0 + 1) < (unsigned)H;
    s.vx0 = (unsigned)s.x0 < (unsigned)W;
    s.vx1 = (unsigned)(s.x0 + 1) < (unsigned)W;
    return s;
}

// Corner offsets/weights with the mask value `m` folded into the weights.
// `cs` is the channel stride of xt (G*Cgp elements per pixel).
__device__ __forceinline__ Corners make_corners(const SamplePos &s, float m, int W, int cs) {
    Corners c;
    const float hy = 1.0f - s.ly, hx = 1.0f - s.lx;
    const bool v00 = s.vy0 && s.vx0, v01 = s.vy0 && s.vx1;
    const bool v10 = s.vy1 && s.vx0, v11 = s.vy1 && s.vx1;
    const int base = (s.y0 * W + s.x0) * cs;
    c.off[0] = v00 ? base : 0;
    c.off[1] = v01 ? base + cs : 0;
    c.off[2] = v10 ? base + W * cs : 0;
    c.off[3] = v11 ? base + (W + 1) * cs : 0;
    c.w[0] = v00 ? hy * hx * m : 0.0f;
    c.w[1] = v01 ? hy * s.lx * m : 0.0f;
    c.w[2] = v10 ? s.ly * hx * m : 0.0f;
    c.w[3] = v11 ? s.ly * s.lx * m : 0.0f;
    return c;
}

__host__ __device__ constexpr inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Number of XCDs of an MI355X; workgroup ids are dispatched round-robin over them.
constexpr int kXcds = 8;

// Bijection on [0, n): workgroup id -> work item such that the ids dispatched
// to one XCD (id % 8 == x) receive one contiguous range of work items.
__device__ __forceinline__ int xcd_remap(int id, int n) {
    const int x = id % kXcds, slot = id / kXcds;
    const int q = n / kXcds, r = n % kXcds;
    return x * q + (x < r ? x : r) + slot;
}
__host__ __device__ constexpr inline int round_up(int a, int b) { return ceil_div(a, b) * b; }

// Buffer -> LDS copy of 16 bytes per lane: lane i's 16 bytes at byte offset
// `off` of the buffer resource land at LDS byte lds + 16*i (lds is
// wave-uniform; an offset at or past the resource's size reads zeros).
// Written as inline assembly so that the compiler does not make later LDS
// reads wait for it (it cannot tell which LDS bytes it writes); a kernel
// waits for it explicitly (s_waitcnt vmcnt(0)) before the barrier or flag
// after which the bytes are read, and the bytes it overwrites were last read
// before an earlier barrier.  (A volatile asm statement stays between the
// barriers around it; without a memory clobber, LDS reads of other buffers
// may be scheduled across it.)  M0 holds the LDS base and is set right
// before the load.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, int off, unsigned lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds"
                 :
                 : "v"(off), "s"(lds), "s"(rs)
                 : "m0");
}
#pragma clang diagnostic pop
// LDS byte address of a __shared__ object.
__device__ __forceinline__ unsigned lds_addr(const void *p) {
    return (unsigned)(size_t)(__attribute__((address_space(3))) const void *)p;
}

}  // namespace dcn2
