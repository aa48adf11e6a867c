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

// Packs 16/sizeof(T) floats into one 16-byte register of T (round to nearest even).
template <typename T> __device__ __forceinline__ uint4 pack16(const float *v) {
    constexpr int E = 16 / sizeof(T);
    T t[E];
#pragma unroll
    for (int e = 0; e < E; ++e) t[e] = (T)v[e];
    return __builtin_bit_cast(uint4, t);
}

// Geometry of one sampling problem (one image at a time).
struct SampleGeo {
    int H, W, kh, kw, sh, sw, ph, pw, dh, dw, G, Cgp, Wo, N, cs, KK;
};

// SPT slots per thread: slot s of thread tid is tid + 512*s.
template <typename T, int SPT> struct Sampler {
    static constexpr int KC = Mma<T>::KC;
    static constexpr int CPS = KC / 4;               // channels per slot
    static constexpr int U4 = CPS * sizeof(T) / 16;  // 16-byte registers per corner (2)
    static_assert(U4 == 2, "a slot covers 32 bytes of one corner");

    int n[SPT], q[SPT], by[SPT], bx[SPT];
    uint4 raw[SPT][4][U4];
    float w[SPT][4];

    // Binds the slots to output pixels n0 + slot/4 of the current image.
    __device__ __forceinline__ void bind(int n0, const SampleGeo &sg, int tid) {
#pragma unroll
        for (int s = 0; s < SPT; ++s) {
            const int slot = tid + s * 512;
            n[s] = n0 + (slot >> 2);
            q[s] = slot & 3;
            const int nn = n[s] < sg.N ? n[s] : 0;
            const int oy = nn / sg.Wo, ox = nn - oy * sg.Wo;
            by[s] = oy * sg.sh - sg.ph;
            bx[s] = ox * sg.sw - sg.pw;
        }
    }

    // Descriptors and corner gathers of chunk `ch` (K order tap, group,
    // channel chunk).  offs/msk/xt point at the current image.
    __device__ __forceinline__ void issue(int ch, const SampleGeo &sg, const T *__restrict__ xt,
                                          const T *__restrict__ offs,
                                          const T *__restrict__ msk) {
        const int cpg = sg.Cgp / KC;
        const int tg = ch / cpg, cc = ch - tg * cpg;
        const int tap = tg / sg.G, g = tg - tap * sg.G;
        const int ki = tap / sg.kw, kj = tap - ki * sg.kw;
#pragma unroll
        for (int s = 0; s < SPT; ++s) {
            Corners c;
            if (n[s] < sg.N) {
                const size_t ob = ((size_t)g * sg.KK + tap) * 2 * sg.N + n[s];
                const float dy = to_f32(offs[ob]);
                const float dx = to_f32(offs[ob + sg.N]);
                const float mv = msk ? to_f32(msk[((size_t)g * sg.KK + tap) * sg.N + n[s]]) : 1.0f;
                const float y = (float)(by[s] + ki * sg.dh) + dy;
                const float x = (float)(bx[s] + kj * sg.dw) + dx;
                c = make_corners(sample_pos(y, x, sg.H, sg.W), mv, sg.W, sg.cs);
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    c.off[k] = 0;
                    c.w[k] = 0.0f;
                }
            }
            const int cbase = g * sg.Cgp + cc * KC + q[s] * CPS;
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
        Unpack<T>::run(raw[s][0][u], v);
#pragma unroll
        for (int e = 0; e < E; ++e) acc[e] = w[s][0] * v[e];
#pragma unroll
        for (int k = 1; k < 4; ++k) {
            Unpack<T>::run(raw[s][k][u], v);
#pragma unroll
            for (int e = 0; e < E; ++e) acc[e] = fmaf(w[s][k], v[e], acc[e]);
        }
    }
};

}  // namespace dcn2
