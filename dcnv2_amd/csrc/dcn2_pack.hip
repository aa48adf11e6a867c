// Repacking kernels that run ahead of the fused forward/backward.
//
// pack_input : NCHW input -> channels-last xt [B][H*W][G*Cgp] with zeroed
//              padding channels, so a bilinear corner is one contiguous channel
//              vector (16-byte loads) instead of C scattered scalars.  The
//              reference samples NCHW directly, one scalar per thread
//              (com.cu:151-195).
// pack_weight: [Cout][C][kh][kw] -> [Mp][Kp] (or its transpose [Kp][Mp]) with
//              K ordered (tap, group, channel) and zero padding, the operand
//              order of the MFMA A fragments.
#include "dcn2_common.h"
#include "dcn2_kernels.h"
#include "../../include/dcnv2_amd.h"

namespace dcn2 {

// 64 pixels x 32 padded channels per block, transposed through LDS.
template <typename T>
__global__ __launch_bounds__(256) void pack_input_kernel(const T *__restrict__ in,
                                                         T *__restrict__ xt, int C, int HW,
                                                         int Cg, int Cgp, int cs) {
    __shared__ T tile[32][64 + 2];
    const int px0 = blockIdx.x * 64, cp0 = blockIdx.y * 32, b = blockIdx.z;
    const int tid = threadIdx.x;
    {
        const int pl = tid & 63, px = px0 + pl;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int cl = (tid >> 6) + 4 * i;
            const int cp = cp0 + cl;
            const int g = cp / Cgp, ci = cp - g * Cgp;
            T v = (T)0.0f;
            if (ci < Cg && px < HW) v = in[((size_t)b * C + g * Cg + ci) * HW + px];
            tile[cl][pl] = v;
        }
    }
    __syncthreads();
    const int pl = tid >> 2, cq = tid & 3, px = px0 + pl;
    if (px < HW) {
        T vals[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) vals[k] = tile[cq * 8 + k][pl];
        T *dst = xt + ((size_t)b * HW + px) * cs + cp0 + cq * 8;
        if constexpr (sizeof(T) == 2) {
            *reinterpret_cast<uint4 *>(dst) = __builtin_bit_cast(uint4, vals);
        } else {
            const uint4 *src = reinterpret_cast<const uint4 *>(vals);
            reinterpret_cast<uint4 *>(dst)[0] = src[0];
            reinterpret_cast<uint4 *>(dst)[1] = src[1];
        }
    }
}

// One thread per packed element.  layout 0 (forward): MFMA A-fragment order,
// dst[((rb*nch + ch)*nks + ks)*64 + lane][e] holds W'[32*rb + lane%32]
// [ch*kc + ks*kstep + (lane/32)*kpl + e], so one wave's fragment load is one
// contiguous run; layout 1 (backward): the same for the transpose W'^T (rows
// k, reduction m): dst[((kb*(Mp/kstep) + ms)*64 + lane)][e] holds
// W'[ms*kstep + (lane/32)*kpl + e][32*kb + lane%32].
// The first nch threads also write the chunk table: for chunk ch of the K
// order (tap, group, channel chunk of kc channels) tab[ch] = {offset/mask
// plane g*KK + tap, row term ki*dh, column term kj*dw, channel base
// g*Cgp + cc*kc}; the sampling kernels read it with scalar loads instead of
// dividing the chunk index every step.
template <typename T>
__global__ __launch_bounds__(256) void pack_weight_kernel(const T *__restrict__ w,
                                                          T *__restrict__ dst, int4 *__restrict__ tab,
                                                          int Cout, int C, int KK, int kw, int dh,
                                                          int dw, int G, int Cg, int Cgp, int kc,
                                                          int kstep, int kpl, int Mp, int Kp,
                                                          int transpose) {
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    const int nch = Kp / kc;
    if (tab && idx < nch) {
        const int cpg = Cgp / kc;
        const int tg = (int)idx / cpg, cc = (int)idx - tg * cpg;
        const int tap = tg / G, g = tg - tap * G;
        const int ki = tap / kw, kj = tap - ki * kw;
        tab[idx] = make_int4(g * KK + tap, ki * dh, kj * dw, g * Cgp + cc * kc);
    }
    if (idx >= (long)Mp * Kp) return;
    int m, k;
    if (transpose) {
        const int nms = Mp / kstep;
        const int e = (int)(idx % kpl);
        long r = idx / kpl;
        const int lane = (int)(r % 64);
        r /= 64;
        const int ms = (int)(r % nms);
        const int kb = (int)(r / nms);
        k = kb * 32 + (lane & 31);
        m = ms * kstep + (lane >> 5) * kpl + e;
    } else {
        // decompose the fragment-order index
        const int nks = kc / kstep;
        const int e = (int)(idx % kpl);
        long r = idx / kpl;
        const int lane = (int)(r % 64);
        r /= 64;
        const int ks = (int)(r % nks);
        r /= nks;
        const int ch = (int)(r % nch);
        const int rb = (int)(r / nch);
        m = rb * 32 + (lane & 31);
        k = ch * kc + ks * kstep + (lane >> 5) * kpl + e;
    }
    const int gc = G * Cgp;
    const int tap = k / gc, r = k - tap * gc;
    const int g = r / Cgp, c = r - g * Cgp;
    T v = (T)0.0f;
    if (m < Cout && c < Cg) v = w[((size_t)m * C + g * Cg + c) * KK + tap];
    dst[idx] = v;
}

template <typename T>
static hipError_t pack_input_t(const Geo &g, const void *input, void *xt, hipStream_t s) {
    const int HW = g.H * g.W;
    dim3 grid(ceil_div(HW, 64), g.cs / 32, g.B);
    pack_input_kernel<T><<<grid, 256, 0, s>>>((const T *)input, (T *)xt, g.C, HW, g.Cg, g.Cgp,
                                              g.cs);
    return hipGetLastError();
}

hipError_t launch_pack_input(const Geo &g, const void *input, void *xt, hipStream_t s) {
    if (g.B == 0) return hipSuccess;
    switch (g.dtype) {
    case DCN2_F16: return pack_input_t<f16>(g, input, xt, s);
    case DCN2_BF16: return pack_input_t<bf16>(g, input, xt, s);
    default: return pack_input_t<float>(g, input, xt, s);
    }
}

template <typename T>
static hipError_t pack_weight_t(const Geo &g, const void *w, void *dst, void *tab, bool tr,
                                hipStream_t s) {
    const long total = (long)g.Mp * g.Kp;
    pack_weight_kernel<T><<<(unsigned)((total + 255) / 256), 256, 0, s>>>(
        (const T *)w, (T *)dst, (int4 *)tab, g.Cout, g.C, g.KK, g.kw, g.dh, g.dw, g.G, g.Cg,
        g.Cgp, g.KC, g.dtype == DCN2_F32 ? 2 : 16, g.dtype == DCN2_F32 ? 1 : 8, g.Mp, g.Kp,
        tr ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_pack_weight(const Geo &g, const void *weight, void *wp, void *tab,
                              bool transpose, hipStream_t s) {
    switch (g.dtype) {
    case DCN2_F16: return pack_weight_t<f16>(g, weight, wp, tab, transpose, s);
    case DCN2_BF16: return pack_weight_t<bf16>(g, weight, wp, tab, transpose, s);
    default: return pack_weight_t<float>(g, weight, wp, tab, transpose, s);
    }
}

}  // namespace dcn2
