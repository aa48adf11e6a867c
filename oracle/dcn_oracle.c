/*
 * CPU oracle for modulated deformable convolution v2 (DCNv2).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path (dcnv2_amd/, the
 * C-ABI library, the drop-in modules) may link, import or call this file.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * always as the checker or as the timed CPU baseline, never as a fallback.
 *
 * This is a scalar restatement of the reference's algorithm with the semantics
 * of torchvision.ops.deform_conv2d(..., mask=...), which the reference
 * documents as its comparator.  It is compiled twice from this one source:
 * REAL=double (suffix _f64, used for parity) and REAL=float (suffix _f32, the
 * CPU baseline that bench.py times).
 *
 * Layouts (all NCHW, contiguous):
 *   input  [B, C, H, W]
 *   weight [Cout, C/WG, kh, kw]          WG weight groups (torchvision groups)
 *   offset [B, G*kh*kw*2, Hout, Wout]   channel (g*kh*kw + k)*2 + {0: dy, 1: dx}
 *   mask   [B, G*kh*kw, Hout, Wout]     channel  g*kh*kw + k   (may be NULL = all 1)
 *   bias   [Cout]                       (may be NULL = all 0)
 *   output [B, Cout, Hout, Wout]
 * with Hout = (H + 2*ph - (dh*(kh-1)+1)) / sh + 1 (likewise Wout), tap
 * k = i*kw + j, input channel c belonging to offset group g = c / (C/G), and
 * output channel m reading only the C/WG input channels of its weight group
 * m / (Cout/WG), as torchvision's deform_conv2d splits its GEMM per group.
 *
 * Function-by-function provenance (reference = /root/reference):
 *   bilinear()        com.cu:119-148 (dcn_bilinear_cuda) plus the in-range test
 *                     of com.cu:187 / com.cu:691.
 *   coord_weight()    com.cu:388-429 (dmcn_get_coordinate_weight_cuda).  With
 *                     ref_boundary=0 it follows torchvision, which has no early
 *                     exit: at a sample exactly on y == -1 or x == -1 one corner
 *                     row/column is in range and the derivative is non-zero.
 *                     ref_boundary=1 reproduces com.cu:392-396 exactly.
 *   sample position   com.cu:176-185 (y = oy*sh - ph + i*dh + dy), with the
 *                     dilation term the reference omits (com.cu:184-185).
 *                     pos_f32=1 rounds that sum to float as the reference
 *                     (com.cu:184, float arithmetic) and torchvision on fp32
 *                     tensors do; pos_f32=0 keeps it exact.  The rounding can
 *                     move a sample lying within one float ulp of an integer
 *                     across it, which changes floor() and hence the one-sided
 *                     grad_offset there, so parity runs against a float32
 *                     implementation use pos_f32=1.
 *   forward           com.cu:151-195 (im2col) + com.cu:46-117 (GEMM + bias),
 *                     computed per output row without materialising columns.
 *   backward          com.cu:733-848: column gradient Wt*gO (com.cu:789-793),
 *                     grad_offset/grad_mask (com.cu:431-501), grad_input
 *                     scatter (com.cu:553-609, the 5x5 neighbourhood test with
 *                     |y-yp| < 1 and the tent weight of com.cu:526-550),
 *                     re-sampled columns for grad_weight (com.cu:637-706,
 *                     829-830) and grad_bias (com.cu:833-835).  Offset groups
 *                     are indexed b*G + g as torchvision does, not b + g
 *                     (com.cu:456-458, a reference bug for G > 1).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#ifndef REAL
#define REAL double
#endif
#define CAT2(a, b) a##b
#define CAT(a, b) CAT2(a, b)
#define FN(name) CAT(name, SUFFIX)

/* Value of channel plane `im` (H x W) at fractional (y, x); 0 outside the open
 * box (-1, H) x (-1, W); corners outside [0,H-1]x[0,W-1] contribute 0.
 * com.cu:119-148 and the range test at com.cu:187. */
static REAL FN(bilinear_)(const REAL *im, int H, int W, REAL y, REAL x) {
    if (!(y > -1 && x > -1 && y < H && x < W)) return 0;
    int y0 = (int)floor(y), x0 = (int)floor(x);
    int y1 = y0 + 1, x1 = x0 + 1;
    REAL ly = y - y0, lx = x - x0, hy = 1 - ly, hx = 1 - lx;
    REAL v1 = (y0 >= 0 && x0 >= 0) ? im[y0 * W + x0] : 0;
    REAL v2 = (y0 >= 0 && x1 <= W - 1) ? im[y0 * W + x1] : 0;
    REAL v3 = (y1 <= H - 1 && x0 >= 0) ? im[y1 * W + x0] : 0;
    REAL v4 = (y1 <= H - 1 && x1 <= W - 1) ? im[y1 * W + x1] : 0;
    return hy * hx * v1 + hy * lx * v2 + ly * hx * v3 + ly * lx * v4;
}

/* d(bilinear)/dy (dir 0) or d/dx (dir 1), one-sided through floor().
 * com.cu:388-429; see the header for ref_boundary. */
static REAL FN(coord_weight_)(const REAL *im, int H, int W, REAL y, REAL x, int dir,
                              int ref_boundary) {
    if (ref_boundary && (y <= -1 || y >= H || x <= -1 || x >= W)) return 0;
    int y0 = (int)floor(y), x0 = (int)floor(x);
    int y1 = y0 + 1, x1 = x0 + 1;
    int vy0 = y0 >= 0 && y0 < H, vy1 = y1 >= 0 && y1 < H;
    int vx0 = x0 >= 0 && x0 < W, vx1 = x1 >= 0 && x1 < W;
    REAL v00 = (vy0 && vx0) ? im[y0 * W + x0] : 0;
    REAL v01 = (vy0 && vx1) ? im[y0 * W + x1] : 0;
    REAL v10 = (vy1 && vx0) ? im[y1 * W + x0] : 0;
    REAL v11 = (vy1 && vx1) ? im[y1 * W + x1] : 0;
    if (dir == 0) {
        REAL lx = x - x0;
        return lx * (v11 - v01) + (1 - lx) * (v10 - v00);
    }
    REAL ly = y - y0;
    return ly * (v11 - v10) + (1 - ly) * (v01 - v00);
}

static REAL FN(pos_)(int base, REAL off, int pos_f32) {
    if (pos_f32) return (REAL)((float)base + (float)off);
    return (REAL)base + off;
}

static int FN(out_size_)(int in, int k, int s, int p, int d) {
    return (in + 2 * p - (d * (k - 1) + 1)) / s + 1;
}

/* Forward.  Returns 0 on success, -1 on invalid arguments. */
int FN(oracle_dcn_forward)(const REAL *input, const REAL *weight, const REAL *offset,
                           const REAL *mask, const REAL *bias, int B, int C, int H, int W,
                           int Cout, int kh, int kw, int sh, int sw, int ph, int pw, int dh,
                           int dw, int G, int WG, REAL *out, int pos_f32, int nthreads) {
    if (B < 0 || C <= 0 || H <= 0 || W <= 0 || Cout <= 0 || kh <= 0 || kw <= 0 || sh <= 0 ||
        sw <= 0 || ph < 0 || pw < 0 || dh <= 0 || dw <= 0 || G <= 0 || C % G || WG <= 0 ||
        C % WG || Cout % WG)
        return -1;
    const int Ho = FN(out_size_)(H, kh, sh, ph, dh), Wo = FN(out_size_)(W, kw, sw, pw, dw);
    if (Ho <= 0 || Wo <= 0) return -1;
    const int KK = kh * kw, CK = C * KK, Cg = C / G, CKw = (C / WG) * KK;
    const long N = (long)Ho * Wo;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
#pragma omp parallel
    {
        REAL *col = (REAL *)malloc(sizeof(REAL) * (size_t)CK * Wo);
#pragma omp for schedule(dynamic)
        for (long t = 0; t < (long)B * Ho; ++t) {
            const int b = (int)(t / Ho), oy = (int)(t % Ho);
            /* columns for this output row: col[(c*KK + k)*Wo + ox] */
            for (int c = 0; c < C; ++c) {
                const int g = c / Cg;
                const REAL *im = input + ((size_t)b * C + c) * H * W;
                for (int k = 0; k < KK; ++k) {
                    const int i = k / kw, j = k % kw;
                    const REAL *offy = offset + (((size_t)b * G + g) * KK * 2 + 2 * k) * N + (size_t)oy * Wo;
                    const REAL *offx = offy + N;
                    const REAL *mk = mask ? mask + (((size_t)b * G + g) * KK + k) * N + (size_t)oy * Wo : NULL;
                    REAL *dst = col + ((size_t)c * KK + k) * Wo;
                    for (int ox = 0; ox < Wo; ++ox) {
                        REAL y = FN(pos_)(oy * sh - ph + i * dh, offy[ox], pos_f32);
                        REAL x = FN(pos_)(ox * sw - pw + j * dw, offx[ox], pos_f32);
                        REAL m = mk ? mk[ox] : (REAL)1;
                        dst[ox] = m * FN(bilinear_)(im, H, W, y, x);
                    }
                }
            }
            for (int m = 0; m < Cout; ++m) {
                REAL *o = out + (((size_t)b * Cout + m) * Ho + oy) * Wo;
                const REAL bv = bias ? bias[m] : 0;
                for (int ox = 0; ox < Wo; ++ox) o[ox] = bv;
                /* weight group of m: columns [ck0, ck0 + CKw) */
                const int ck0 = (m / (Cout / WG)) * CKw;
                const REAL *wr = weight + (size_t)m * CKw - ck0;
                for (int ck = ck0; ck < ck0 + CKw; ++ck) {
                    const REAL wv = wr[ck];
                    const REAL *cr = col + (size_t)ck * Wo;
                    for (int ox = 0; ox < Wo; ++ox) o[ox] += wv * cr[ox];
                }
            }
        }
        free(col);
    }
    return 0;
}

/* Backward.  All five gradients are overwritten (not accumulated).  grad_mask
 * may be NULL only when mask is NULL; grad_bias may be NULL.  Returns 0 on
 * success, -1 on invalid arguments, -2 on allocation failure. */
int FN(oracle_dcn_backward)(const REAL *input, const REAL *weight, const REAL *offset,
                            const REAL *mask, const REAL *grad_out, int B, int C, int H, int W,
                            int Cout, int kh, int kw, int sh, int sw, int ph, int pw, int dh,
                            int dw, int G, int WG, REAL *grad_input, REAL *grad_weight,
                            REAL *grad_bias, REAL *grad_offset, REAL *grad_mask,
                            int ref_boundary, int pos_f32, int nthreads) {
    if (B < 0 || C <= 0 || H <= 0 || W <= 0 || Cout <= 0 || kh <= 0 || kw <= 0 || sh <= 0 ||
        sw <= 0 || ph < 0 || pw < 0 || dh <= 0 || dw <= 0 || G <= 0 || C % G || WG <= 0 ||
        C % WG || Cout % WG)
        return -1;
    const int Ho = FN(out_size_)(H, kh, sh, ph, dh), Wo = FN(out_size_)(W, kw, sw, pw, dw);
    if (Ho <= 0 || Wo <= 0) return -1;
    const int KK = kh * kw, CK = C * KK, Cg = C / G, CKw = (C / WG) * KK, mpg = Cout / WG;
    const long N = (long)Ho * Wo;
    memset(grad_input, 0, sizeof(REAL) * (size_t)B * C * H * W);
    memset(grad_weight, 0, sizeof(REAL) * (size_t)Cout * CKw);
    memset(grad_offset, 0, sizeof(REAL) * (size_t)B * G * KK * 2 * N);
    if (grad_mask) memset(grad_mask, 0, sizeof(REAL) * (size_t)B * G * KK * N);
    if (grad_bias) {
        /* com.cu:833-835: grad_bias = sum over batch and pixels of grad_out */
        for (int m = 0; m < Cout; ++m) {
            REAL s = 0;
            for (int b = 0; b < B; ++b) {
                const REAL *go = grad_out + ((size_t)b * Cout + m) * N;
                for (long p = 0; p < N; ++p) s += go[p];
            }
            grad_bias[m] = s;
        }
    }
    int nt = 1;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
    nt = omp_get_max_threads();
#endif
    REAL *gw_part = (REAL *)calloc((size_t)nt * Cout * CKw, sizeof(REAL));
    if (!gw_part) return -2;
    /* one image per task: grad_input of image b is written by one thread only */
#pragma omp parallel
    {
        int tid = 0;
#ifdef _OPENMP
        tid = omp_get_thread_num();
#endif
        REAL *gw = gw_part + (size_t)tid * Cout * CKw;
        REAL *cg = (REAL *)malloc(sizeof(REAL) * (size_t)CK * Wo);  /* column gradient */
        REAL *cs = (REAL *)malloc(sizeof(REAL) * (size_t)CK * Wo);  /* re-sampled columns */
#pragma omp for schedule(dynamic)
        for (int b = 0; b < B; ++b) {
            for (int oy = 0; oy < Ho; ++oy) {
                /* column gradient, com.cu:789-793: cg[ck][ox] = sum_m W[m][ck] gO[b][m][oy][ox] */
                memset(cg, 0, sizeof(REAL) * (size_t)CK * Wo);
                for (int m = 0; m < Cout; ++m) {
                    const REAL *go = grad_out + (((size_t)b * Cout + m) * Ho + oy) * Wo;
                    const int ck0 = (m / mpg) * CKw; /* m's weight group */
                    const REAL *wr = weight + (size_t)m * CKw - ck0;
                    for (int ck = ck0; ck < ck0 + CKw; ++ck) {
                        const REAL wv = wr[ck];
                        REAL *d = cg + (size_t)ck * Wo;
                        for (int ox = 0; ox < Wo; ++ox) d[ox] += wv * go[ox];
                    }
                }
                for (int c = 0; c < C; ++c) {
                    const int g = c / Cg;
                    const REAL *im = input + ((size_t)b * C + c) * H * W;
                    REAL *gim = grad_input + ((size_t)b * C + c) * H * W;
                    for (int k = 0; k < KK; ++k) {
                        const int i = k / kw, j = k % kw;
                        const size_t obase = (((size_t)b * G + g) * KK * 2 + 2 * k) * N + (size_t)oy * Wo;
                        const size_t mbase = (((size_t)b * G + g) * KK + k) * N + (size_t)oy * Wo;
                        const REAL *cgr = cg + ((size_t)c * KK + k) * Wo;
                        REAL *csr = cs + ((size_t)c * KK + k) * Wo;
                        for (int ox = 0; ox < Wo; ++ox) {
                            const REAL y = FN(pos_)(oy * sh - ph + i * dh, offset[obase + ox], pos_f32);
                            const REAL x = FN(pos_)(ox * sw - pw + j * dw, offset[obase + N + ox], pos_f32);
                            const REAL mv = mask ? mask[mbase + ox] : (REAL)1;
                            const REAL cgv = cgr[ox];
                            const REAL val = FN(bilinear_)(im, H, W, y, x);
                            csr[ox] = mv * val;
                            /* grad_offset / grad_mask, com.cu:486-492 */
                            grad_offset[obase + ox] +=
                                mv * cgv * FN(coord_weight_)(im, H, W, y, x, 0, ref_boundary);
                            grad_offset[obase + N + ox] +=
                                mv * cgv * FN(coord_weight_)(im, H, W, y, x, 1, ref_boundary);
                            if (grad_mask) grad_mask[mbase + ox] += cgv * val;
                            /* grad_input scatter, com.cu:590-607 */
                            const REAL top = cgv * mv;
                            const int yt = (int)y, xt = (int)x; /* truncation, as com.cu:591-592 */
                            for (int dy = -2; dy <= 2; ++dy) {
                                const int yp = yt + dy;
                                if (yp < 0 || yp >= H || fabs(y - yp) >= 1) continue;
                                for (int dx = -2; dx <= 2; ++dx) {
                                    const int xp = xt + dx;
                                    if (xp < 0 || xp >= W || fabs(x - xp) >= 1) continue;
                                    gim[yp * W + xp] += top * (1 - fabs(y - yp)) * (1 - fabs(x - xp));
                                }
                            }
                        }
                    }
                }
                /* grad_weight, com.cu:829-830: gW[m][ck] += sum_ox gO[m][ox] * cols[ck][ox] */
                for (int m = 0; m < Cout; ++m) {
                    const REAL *go = grad_out + (((size_t)b * Cout + m) * Ho + oy) * Wo;
                    const int ck0 = (m / mpg) * CKw;
                    REAL *gwr = gw + (size_t)m * CKw - ck0;
                    for (int ck = ck0; ck < ck0 + CKw; ++ck) {
                        const REAL *csr = cs + (size_t)ck * Wo;
                        REAL s = 0;
                        for (int ox = 0; ox < Wo; ++ox) s += go[ox] * csr[ox];
                        gwr[ck] += s;
                    }
                }
            }
        }
        free(cg);
        free(cs);
    }
    for (int t = 0; t < nt; ++t) {
        const REAL *src = gw_part + (size_t)t * Cout * CKw;
        for (size_t e = 0; e < (size_t)Cout * CKw; ++e) grad_weight[e] += src[e];
    }
    free(gw_part);
    return 0;
}
