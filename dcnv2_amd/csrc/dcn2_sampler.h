// Mask-modulated bilinear sampler shared by the forward kernel and the
// grad_weight kernel (both need the sampled column chunk in LDS).
//
// A sampling slot is (pixel, quarter of a KC-channel chunk): 4 adjacent lanes
// cover one pixel's KC channels, so each bilinear corner of a pixel is read as
// one contiguous KC*sizeof(T)-byte run of the channels-last input (two 16-byte
// loads per lane).  The value follows reference com.cu:119-195:
//   col[c] = mask * sum_q w_q * input[c, corner_q]
// with the corner weights of the floor-based bilinear rule and zero for a
// corner outside the image; blend arithmetic is fp32.
#pragma once

#include "dcn2_common.h"

namespace dcn2 {

template <typename T> struct Unpack;
template <> struct Unpack<f16> {
    static constexpr int E = 8;
    static __device__ __forceinline__ void run(uint4 r, float *o) {
        const f16x8 h = __builtin_bit_cast(f16x8, r);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (float)h[e];
    }
};
template <> struct Unpack<bf16> {
    static constexpr int E = 8;
    static __device__ __forceinline__ void run(uint4 r, float *o) {
        const uint32_t u[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            o[2 * e] = __uint_as_float(u[e] << 16);
            o[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
        }
    }
};
template <> struct Unpack<float> {
    static constexpr int E = 4;
    static __device__ __forceinline__ void run(uint4 r, float *o) {
        o[0] = __uint_as_float(r.x);
        o[1] = __uint_as_float(r.y);
        o[2] = __uint_as_float(r.z);
        o[3] = __uint_as_float(r.w);
    }
};

// Packs 16/sizeof(T) floats into one 16-byte register of T (round to nearest
// even).  2-byte types convert pairs (one v_cvt_pk_{f16,bf16}_f32 each).
template <typename T> __device__ __forceinline__ uint4 pack16(const float *v) {
    constexpr int E = 16 / sizeof(T);
    if constexpr (sizeof(T) == 2) {
        typedef float f2 __attribute__((ext_vector_type(2)));
        typedef T t2 __attribute__((ext_vector_type(2)));
        t2 t[E / 2];
#pragma unroll
        for (int e = 0; e < E / 2; ++e) t[e] = __builtin_convertvector(f2{v[2 * e], v[2 * e + 1]}, t2);
        return __builtin_bit_cast(uint4, t);
    } else {
        T t[E];
#pragma unroll
        for (int e = 0; e < E; ++e) t[e] = (T)v[e];
        return __builtin_bit_cast(uint4, t);
    }
}

// Geometry of one sampling problem (one image at a time).
struct SampleGeo {
    int H, W, kh, kw, sh, sw, ph, pw, dh, dw, G, Cgp, Wo, N, cs, KK;
    int msk_logit;  // mask buffer holds logits (see mask_value)
};

// Raw offset/mask bits and output-pixel coordinates of one chunk for the SPT
// slots of a thread.  Kept unconverted so that the load can be issued one
// pipeline step before its first use without forcing an early wait.  A slot
// past the last pixel has by == kNoPixel.
constexpr int kNoPixel = -2147483647 - 1;
template <typename T, int SPT> struct SlotOM {
    int by[SPT], bx[SPT];
    T dy[SPT], dx[SPT], m[SPT];
};

// Chunk table entry (written by pack_weight_kernel): x = offset/mask plane
// g*KK + tap, y = ki*dh, z = kj*dw, w = first channel g*Cgp + cc*KC of the
// chunk inside a pixel's channel vector.
typedef int4 ChunkEnt;

// SPT slots per thread: slot s of thread tid is tid + 512*s, covering output
// pixel n0 + slot/4 and channel quarter slot%4 of the chunk.  MASK: a mask
// tensor is present (else every mask value is 1).
template <typename T, int SPT, bool MASK> struct Sampler {
    static constexpr int KC = Mma<T>::KC;
    static constexpr int CPS = KC / 4;               // channels per slot
    static constexpr int U4 = CPS * sizeof(T) / 16;  // 16-byte registers per corner (2)
    static_assert(U4 == 2, "a slot covers 32 bytes of one corner");

    int q;  // channel quarter of every slot of this thread (512 % 4 == 0)
    uint4 raw[SPT][4][U4];
    float w[SPT][4];

    __device__ __forceinline__ void init(int tid) { q = tid & 3; }

    // Offset/mask bits of plane `plane` for the pixels n0 + slot/4 of the
    // image whose offset/mask planes start at offs/msk.
    __device__ __forceinline__ void load_om(int n0, int plane, const SampleGeo &sg, int tid,
                                            const T *__restrict__ offs,
                                            const T *__restrict__ msk,
                                            SlotOM<T, SPT> &om) const {
#pragma unroll
        for (int s = 0; s < SPT; ++s) {
            const int n = n0 + ((tid + s * 512) >> 2);
            const int nn = n < sg.N ? n : 0;
            const int oy = nn / sg.Wo, ox = nn - oy * sg.Wo;
            om.by[s] = n < sg.N ? oy * sg.sh - sg.ph : kNoPixel;
            om.bx[s] = ox * sg.sw - sg.pw;
            const size_t ob = (size_t)plane * 2 * sg.N + nn;
            om.dy[s] = offs[ob];
            om.dx[s] = offs[ob + sg.N];
            if constexpr (MASK) om.m[s] = msk[(size_t)plane * sg.N + nn];
        }
    }

    // Descriptors and corner gathers of the chunk `e` from `om`.
    __device__ __forceinline__ void issue(const ChunkEnt &e, const SampleGeo &sg,
                                          const T *__restrict__ xt, const SlotOM<T, SPT> &om) {
#pragma unroll
        for (int s = 0; s < SPT; ++s) {
            const float y = (float)(om.by[s] + e.y) + to_f32(om.dy[s]);
            const float x = (float)(om.bx[s] + e.z) + to_f32(om.dx[s]);
            float mv = 1.0f;
            if constexpr (MASK) mv = mask_value(to_f32(om.m[s]), sg.msk_logit);
            mv = om.by[s] != kNoPixel ? mv : 0.0f;  // pixels past N sample 0
            const Corners c = make_corners(sample_pos(y, x, sg.H, sg.W), mv, sg.W, sg.cs);
            const int cbase = e.w + q * CPS;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                w[s][k] = c.w[k];
                const uint4 *src = reinterpret_cast<const uint4 *>(xt + c.off[k] + cbase);
#pragma unroll
                for (int u = 0; u < U4; ++u) raw[s][k][u] = src[u];
            }
        }
    }

    // Blended values of 16-byte register u (E channels) of slot s.
    __device__ __forceinline__ void blend(int s, int u, float *acc) const {
        constexpr int E = Unpack<T>::E;
        float v[E];
#pragma unroll
        for (int e = 0; e < E; ++e) acc[e] = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            Unpack<T>::run(raw[s][k][u], v);
#pragma unroll
            for (int e = 0; e < E; ++e) acc[e] = fmaf(w[s][k], v[e], acc[e]);
        }
    }
};

}  // namespace dcn2
