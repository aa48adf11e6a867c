// extern "C" entry points of libdcnv2_amd.so (declared in include/dcnv2_amd.h).
//
// Host-side work of the reference's MyDCN_forward / MyDCN_backward
// (com.cu:198-272, 733-848): argument validation, output-shape math, scratch
// carving and the launch sequence.  Scratch comes from the caller's workspace
// (the Python layer allocates it from torch's caching allocator), never from
// hipMalloc, and every launch goes to the caller's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/dcnv2_amd.h"
#include "dcn2_common.h"
#include "dcn2_kernels.h"
#include "dcn2_profile.h"

namespace dcn2 {

static thread_local std::string g_last_error;

// process-wide options (dcn2_set_option)
static std::atomic<long long> g_opt_slice_bytes{DCN2_BWD_SLICE_BYTES_DEFAULT};
static std::atomic<int> g_opt_fused{-1}, g_opt_push{-1};

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Validates `d` and derives the packing geometry.  Returns DCN2_OK or an error.
int make_geo(const dcn2_desc *d, Geo &g) {
    if (!d) return fail(DCN2_EINVAL, "dcn2: null descriptor");
    g.B = d->batch;
    g.C = d->in_channels;
    g.H = d->height;
    g.W = d->width;
    g.Cout = d->out_channels;
    g.kh = d->kernel_h;
    g.kw = d->kernel_w;
    g.sh = d->stride_h;
    g.sw = d->stride_w;
    g.ph = d->pad_h;
    g.pw = d->pad_w;
    g.dh = d->dilation_h;
    g.dw = d->dilation_w;
    g.G = d->deformable_groups;
    g.dtype = d->dtype;
    g.WG = d->weight_groups == 0 ? 1 : d->weight_groups;
    g.nhwc = d->input_layout;
    if (g.nhwc != DCN2_NCHW && g.nhwc != DCN2_NHWC)
        return fail(DCN2_EINVAL, "dcn2: unsupported input_layout %d", g.nhwc);
    g.out_nhwc = d->output_layout;
    if (g.out_nhwc != DCN2_NCHW && g.out_nhwc != DCN2_NHWC)
        return fail(DCN2_EINVAL, "dcn2: unsupported output_layout %d", g.out_nhwc);
    if (g.dtype != DCN2_F32 && g.dtype != DCN2_F16 && g.dtype != DCN2_BF16)
        return fail(DCN2_EINVAL, "dcn2: unsupported dtype code %d", g.dtype);
    if (g.B < 0 || g.C <= 0 || g.H <= 0 || g.W <= 0 || g.Cout <= 0)
        return fail(DCN2_EINVAL, "dcn2: invalid shape B=%d C=%d H=%d W=%d Cout=%d", g.B, g.C,
                    g.H, g.W, g.Cout);
    if (g.kh <= 0 || g.kw <= 0 || g.sh <= 0 || g.sw <= 0 || g.dh <= 0 || g.dw <= 0 ||
        g.ph < 0 || g.pw < 0)
        return fail(DCN2_EINVAL,
                    "dcn2: invalid kernel/stride/padding/dilation (%d,%d)/(%d,%d)/(%d,%d)/(%d,%d)",
                    g.kh, g.kw, g.sh, g.sw, g.ph, g.pw, g.dh, g.dw);
    if (g.G <= 0 || g.C % g.G != 0)
        return fail(DCN2_EINVAL, "dcn2: in_channels %d not divisible by deformable_groups %d",
                    g.C, g.G);
    if (g.WG <= 0 || g.C % g.WG != 0 || g.Cout % g.WG != 0)
        return fail(DCN2_EINVAL,
                    "dcn2: in_channels %d and out_channels %d not divisible by weight_groups %d",
                    g.C, g.Cout, g.WG);
    g.Cw = g.C / g.WG;
    g.Ho = (g.H + 2 * g.ph - (g.dh * (g.kh - 1) + 1)) / g.sh + 1;
    g.Wo = (g.W + 2 * g.pw - (g.dw * (g.kw - 1) + 1)) / g.sw + 1;
    if (g.H + 2 * g.ph < g.dh * (g.kh - 1) + 1 || g.W + 2 * g.pw < g.dw * (g.kw - 1) + 1 ||
        g.Ho <= 0 || g.Wo <= 0)
        return fail(DCN2_EINVAL, "dcn2: empty output (%d x %d)", g.Ho, g.Wo);
    g.slice_bytes = g_opt_slice_bytes.load(std::memory_order_relaxed);
    g.opt_fused = g_opt_fused.load(std::memory_order_relaxed);
    g.opt_push = g_opt_push.load(std::memory_order_relaxed);
    g.Bs = g.B;
    g.esz = g.dtype == DCN2_F32 ? 4 : 2;
    g.KC = g.dtype == DCN2_F32 ? 32 : 64;
    g.Cg = g.C / g.G;
    g.Cgp = round_up(g.Cg, g.KC);
    g.cs = g.G * g.Cgp;
    g.xt_direct = g.nhwc && g.cs == g.C;
    g.N = g.Ho * g.Wo;
    g.KK = g.kh * g.kw;
    g.BM = g.Cout > 128 ? 256 : 128;
    g.Mp = round_up(g.Cout, g.BM);
    // All in-kernel offsets within one image (and of the packed weights) are
    // 32-bit; the per-image base is 64-bit.
    const long long lim = 0x7fffffffLL;
    const long long Kp = (long long)g.KK * g.cs;
    if ((long long)g.H * g.W * g.cs >= lim || (long long)g.C * g.H * g.W >= lim ||
        (long long)g.Ho * g.Wo * g.Cout >= lim || (long long)g.Ho * g.Wo * 2 * g.G * g.KK >= lim ||
        Kp * g.Mp >= lim || (long long)g.Ho * g.Wo >= lim || g.B > 65535 ||
        (long long)g.B * g.G * g.KK * g.Ho * g.Wo >= lim || g.H > 32767 || g.W > 32767)
        return fail(DCN2_ERANGE, "dcn2: problem exceeds the 32-bit per-image index range");
    g.Kp = (int)Kp;
    // weight-group walk (see Geo::gsplit): every chunk (deformable group dg,
    // channel chunk cc) must lie inside the group q / cpw of its index q in
    // the tap
    g.cpt = g.G * (g.Cgp / g.KC);
    g.cpw = g.cpt;
    g.gsplit = 0;
    if (g.WG > 1 && (g.Cout / g.WG) % 128 == 0 && g.cpt % g.WG == 0) {
        const int cpg = g.Cgp / g.KC, cpw = g.cpt / g.WG;
        bool ok = true;
        for (int q = 0; q < g.cpt && ok; ++q) {
            const int dg = q / cpg, cc = q % cpg;
            const int lo = dg * g.Cg + cc * g.KC;
            const int hi = dg * g.Cg + std::min((cc + 1) * g.KC, g.Cg) - 1;
            ok = lo / g.Cw == hi / g.Cw && lo / g.Cw == q / cpw;
        }
        if (ok) {
            g.gsplit = 1;
            g.cpw = cpw;
        }
    }
    // the forward's sampler addresses one image of xt with 32-bit byte offsets
    // and marks corners outside the image with the offset just past it
    if (((long long)g.H * g.W + 1) * g.cs * g.esz + 256 >= 0x100000000LL)
        return fail(DCN2_ERANGE, "dcn2: one image of %d x %d x %d channels exceeds the 32-bit "
                    "byte range", g.H, g.W, g.cs);
    {
        const GatherGeo gg = gather_geometry(g);
        if (gg.batch_bytes >= gg.max_batch_bytes)
            return fail(DCN2_ERANGE, "dcn2: %d channels per deformable group exceed the "
                        "grad_input gather's row range", g.Cg);
    }
    // separate offset and mask tensors (dcn2_forward / dcn2_backward)
    g.off_bs = 2LL * g.G * g.KK * g.N;
    g.msk_bs = (long long)g.G * g.KK * g.N;
    g.msk_logit = 0;
    g.rw = rw_eligible(g) ? 1 : 0;
    return DCN2_OK;
}

// The predictor-output layout of dcn2_forward_om / dcn2_backward_om: one
// [B, 3*G*KK, Ho, Wo] tensor, offsets in its first 2*G*KK channels and mask
// logits in the rest (the reference's chunk(3) / cat / sigmoid split,
// dcn_v2_mm.py:133-137).  Returns the element offset of the mask channels.
static int use_om_layout(Geo &g, long long &mask_off) {
    if (3LL * g.G * g.KK * g.N >= 0x7fffffffLL)
        return fail(DCN2_ERANGE, "dcn2: offset/mask tensor exceeds the 32-bit per-image index range");
    g.off_bs = g.msk_bs = 3LL * g.G * g.KK * g.N;
    g.msk_logit = 1;
    mask_off = 2LL * g.G * g.KK * g.N;
    return DCN2_OK;
}

FwdWorkspace fwd_workspace(const Geo &g) {
    FwdWorkspace w;
    size_t o = 0;
    w.xt = o;
    if (!g.xt_direct) o += align256((size_t)g.B * g.H * g.W * g.cs * g.esz);
    w.wp = o;
    o += align256((size_t)g.Mp * g.Kp * g.esz);
    w.tab = o;
    o += align256((size_t)(g.Kp / g.KC) * 16);
    w.total = o;
    return w;
}

BwdWorkspace bwd_workspace(const Geo &g0) {
    Geo g = g0;
    g.B = g0.Bs;
    BwdWorkspace w;
    size_t o = 0;
    w.xt = o;
    const size_t xt_bytes = g.xt_direct ? 0 : align256((size_t)g.B * g.H * g.W * g.cs * g.esz);
    o += xt_bytes;
    w.wt = o;
    o += align256((size_t)g.Mp * g.Kp * g.esz);
    w.tab = o;
    o += align256((size_t)(g.Kp / g.KC) * 16);
    const GatherGeo gg = gather_geometry(g);
    w.gi_acc = o;  // (by pixels only: partial sums of buckets of several record batches)
    if (!gg.by_cells) o += align256((size_t)gg.acc_bytes);
    w.gw_acc = o;
    o += align256((size_t)g.Mp * g.Kp * sizeof(float));
    w.gb_acc = o;
    o += align256((size_t)g.Mp * sizeof(float));
    w.cgm = o;
    o += align256((size_t)gg.rows * g.Cgp * gg.row_esz);
    w.rsc = o;
    if (gg.row_scaled) o += align256((size_t)gg.rows * (g.Cgp / 32));
    w.csum = o;  // fp32 corner sums [B][G*KK][N][4] of the fused kernel
    if (fused_bwd_shape(g) && g.Cgp > g.KC) o += align256((size_t)g.B * g.G * g.KK * g.N * 16);
    w.rec = o;
    o += align256((size_t)gg.rows * 12);  // 12-byte sample records
    w.bcnt = o;
    o += align256((size_t)gg.nbuckets * sizeof(int) + 16);
    w.bstart = o;
    o += align256((size_t)(gg.nbuckets + 1) * sizeof(int));
    w.bcur = o;
    o += align256((size_t)gg.nbuckets * sizeof(int));
    w.sidx = o;
    o += align256((size_t)g.B * g.G * g.KK * g.N * sizeof(int));
    // The border rings are written after the last read of xt (the
    // grad_weight kernels and the column-gradient kernels run before the
    // grad_input kernels), so they share xt's bytes when they fit there.
    const size_t ring_bytes = align256((size_t)gg.nbuckets * kGatherRing * g.Cgp * sizeof(float));
    if (ring_bytes <= xt_bytes) {
        w.ring = w.xt;
    } else {
        w.ring = o;
        o += ring_bytes;
    }
    w.total = o;
    return w;
}

// Images per backward slice: the largest count whose workspace fits the
// slice budget (at least one), then evened out over the slices that count
// implies (B = 16 with room for 6 runs as 6 + 5 + 5, not 6 + 6 + 4).
static int bwd_slice_images(const Geo &g) {
    auto bytes = [&](int b) {
        Geo t = g;
        t.Bs = b;
        return bwd_workspace(t).total;
    };
    const size_t budget = (size_t)std::max(1LL, g.slice_bytes);
    if (g.B <= 1 || bytes(g.B) <= budget) return g.B;
    int lo = 1, hi = g.B;  // bytes(lo) fits or lo == 1; bytes(hi) does not
    while (hi - lo > 1) {
        const int mid = lo + (hi - lo) / 2;
        if (bytes(mid) <= budget) lo = mid;
        else hi = mid;
    }
    const int nslices = (g.B + lo - 1) / lo;
    return (g.B + nslices - 1) / nslices;
}

static int check_launch(hipError_t e, const char *what) {
    if (e != hipSuccess)
        return fail(DCN2_ELAUNCH, "dcn2: %s launch failed: %s", what, hipGetErrorString(e));
    return DCN2_OK;
}

int forward_impl(const Geo &g, const void *input, const void *weight, const void *mask,
                 const void *offset, const void *bias, void *output, void *workspace,
                 size_t workspace_bytes, void *stream) {
    int rc = DCN2_OK;
    if (g.B > 0 && (!input || !offset || !output))
        return fail(DCN2_EINVAL, "dcn2_forward: null input/offset/output pointer");
    if (!weight) return fail(DCN2_EINVAL, "dcn2_forward: null weight pointer");
    const FwdWorkspace ws = fwd_workspace(g);
    if (!workspace || workspace_bytes < ws.total || ((uintptr_t)workspace & 255))
        return fail(DCN2_EWORKSPACE,
                    "dcn2_forward: workspace needs %zu bytes at 256-byte alignment (got %zu)",
                    ws.total, workspace_bytes);
    if (g.B == 0) return DCN2_OK;
    // The resident-weight forward stores 16-byte pieces; for an output that is
    // not 16-byte aligned the chunk-streaming kernel runs instead (both read
    // the same channels-last copy).
    Geo gf = g;
    if (gf.rw && ((uintptr_t)output & 15)) gf.rw = 0;
    // a channels-last input whose channels need no padding is read in place
    const bool direct = gf.xt_direct;
    if (direct && ((uintptr_t)input & 15))
        return fail(DCN2_EINVAL, "dcn2_forward: a channels-last input must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    char *base = (char *)workspace;
    const void *xt = direct ? input : base + ws.xt;
    void *wp = base + ws.wp, *tab = base + ws.tab;
    prof_begin(DCN2_STAGE_FWD_PACK, s);
    if ((rc = check_launch(launch_pack(gf, direct ? nullptr : input, (void *)xt, weight, wp, tab,
                                       false, s), "pack")))
        return rc;
    prof_end(DCN2_STAGE_FWD_PACK, s);
    prof_begin(DCN2_STAGE_FWD_MAIN, s);
    if (gf.rw)
        rc = check_launch(launch_forward_rw(gf, xt, wp, offset, mask, bias, output, s), "forward");
    else
        rc = check_launch(launch_forward(gf, xt, wp, tab, offset, mask, bias, output, s), "forward");
    prof_end(DCN2_STAGE_FWD_MAIN, s);
    return rc;
}

static int backward_impl(const Geo &g0, const void *input, const void *weight, const void *mask,
                         const void *offset, const void *grad_output, void *grad_input,
                         void *grad_offset, void *grad_mask, void *grad_weight, void *grad_bias,
                         void *workspace, size_t workspace_bytes, void *stream) {
    int rc = DCN2_OK;

    if (!weight || !grad_weight)
        return fail(DCN2_EINVAL, "dcn2_backward: null weight/grad_weight pointer");
    if (g0.B > 0 && (!input || !offset || !grad_output || !grad_input || !grad_offset))
        return fail(DCN2_EINVAL, "dcn2_backward: null input/offset/grad pointer");
    if ((mask == nullptr) != (grad_mask == nullptr))
        return fail(DCN2_EINVAL, "dcn2_backward: grad_mask must be given exactly when mask is");
    Geo g = g0;
    g.Bs = bwd_slice_images(g0);
    const BwdWorkspace ws = bwd_workspace(g);
    if (!workspace || workspace_bytes < ws.total || ((uintptr_t)workspace & 255))
        return fail(DCN2_EWORKSPACE,
                    "dcn2_backward: workspace needs %zu bytes at 256-byte alignment (got %zu)",
                    ws.total, workspace_bytes);
    if (g.B > 0 && g.xt_direct && ((uintptr_t)input & 15))
        return fail(DCN2_EINVAL, "dcn2_backward: a channels-last input must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    char *base = (char *)workspace;
    void *wt = base + ws.wt, *tab = base + ws.tab;
    // Slices of g.Bs images (the last may hold fewer), each on the same
    // workspace in stream order: its pack launch transposes the slice's input
    // and zeroes the bucket counts (the first one also packs the weight and
    // zeroes the grad_weight / grad_bias accumulators, which every slice adds
    // to); the last slice writes grad_weight / grad_bias.  An empty batch is
    // one slice of no images.
    const size_t esz = g.esz;
    const size_t in_img = (size_t)g.C * g.H * g.W * esz, go_img = (size_t)g.Cout * g.N * esz;
    const size_t off_img = (size_t)g.off_bs * esz, msk_img = (size_t)g.msk_bs * esz;
    int b0 = 0;
    do {
        Geo gs = g;
        gs.B = std::min(g.Bs, g.B - b0);
        gs.Bs = gs.B;
        const bool first = b0 == 0, last = b0 + gs.B >= g.B;
        auto at = [&](const void *ptr, size_t img) -> const char * {
            return ptr ? (const char *)ptr + (size_t)b0 * img : nullptr;
        };
        const void *in_s = at(input, in_img);
        const void *xt = g.xt_direct ? in_s : base + ws.xt;
        const GatherGeo gg = gather_geometry(gs);
        ClearList clr;
        clr.p[0] = (float *)(base + ws.gw_acc);
        clr.n[0] = first ? (size_t)g.Mp * g.Kp : 0;
        clr.p[1] = (float *)(base + ws.gb_acc);
        clr.n[1] = first && grad_bias ? (size_t)g.Mp : 0;
        // (bcnt, bstart and bcur are adjacent: the place pass that scans the
        // counts itself claims rows from bcur = 0)
        clr.p[2] = (float *)(base + ws.bcnt);
        clr.n[2] = gs.B > 0 ? (ws.bcur - ws.bcnt) / sizeof(int) + (size_t)gg.nbuckets : 0;
        clr.p[3] = (float *)(base + ws.csum);
        clr.n[3] = ws.rec > ws.csum && gs.B > 0 ? (size_t)gs.B * g.G * g.KK * g.N * 4 : 0;
        prof_begin(DCN2_STAGE_BWD_PACK, s);
        if ((rc = check_launch(launch_pack(gs, g.xt_direct ? nullptr : in_s, (void *)xt,
                                           first ? weight : nullptr, wt, tab, true, s, &clr),
                               "pack")))
            return rc;
        prof_end(DCN2_STAGE_BWD_PACK, s);
        if ((rc = check_launch(
                 launch_backward(gs, xt, wt, tab, at(offset, off_img), at(mask, msk_img),
                                 at(grad_output, go_img), (void *)at(grad_input, in_img),
                                 (void *)at(grad_offset, off_img), (void *)at(grad_mask, msk_img),
                                 grad_weight, grad_bias, (float *)(base + ws.gi_acc),
                                 (float *)(base + ws.gw_acc), (float *)(base + ws.gb_acc),
                                 base + ws.cgm, base + ws.rsc, (float *)(base + ws.csum), base + ws.rec,
                                 (int *)(base + ws.bcnt),
                                 (int *)(base + ws.bstart), (int *)(base + ws.bcur),
                                 (int *)(base + ws.sidx), (float *)(base + ws.ring), last, s),
                 "backward")))
            return rc;
        b0 += gs.B;
    } while (b0 < g.B);
    return DCN2_OK;
}


}  // namespace dcn2

using namespace dcn2;

extern "C" {

int dcn2_output_shape(const dcn2_desc *d, int32_t *out_h, int32_t *out_w) {
    Geo g;
    const int rc = make_geo(d, g);
    if (rc) return rc;
    if (out_h) *out_h = g.Ho;
    if (out_w) *out_w = g.Wo;
    return DCN2_OK;
}

size_t dcn2_forward_workspace_bytes(const dcn2_desc *d) {
    Geo g;
    if (make_geo(d, g)) return 0;
    return fwd_workspace(g).total;
}

size_t dcn2_backward_workspace_bytes(const dcn2_desc *d) {
    Geo g;
    if (make_geo(d, g)) return 0;
    g.Bs = bwd_slice_images(g);
    return bwd_workspace(g).total;
}

int dcn2_set_option(int option, int64_t value) {
    switch (option) {
    case DCN2_OPT_BWD_SLICE_BYTES:
        if (value < 1) return fail(DCN2_EINVAL, "dcn2_set_option: slice budget %lld < 1", (long long)value);
        g_opt_slice_bytes.store(value, std::memory_order_relaxed);
        return DCN2_OK;
    case DCN2_OPT_BWD_FUSED:
        if (value != -1 && value != 0)
            return fail(DCN2_EINVAL, "dcn2_set_option: DCN2_OPT_BWD_FUSED takes -1 or 0, not %lld",
                        (long long)value);
        g_opt_fused.store((int)value, std::memory_order_relaxed);
        return DCN2_OK;
    case DCN2_OPT_GI_PUSH:
        if (value < -1 || value > 1)
            return fail(DCN2_EINVAL, "dcn2_set_option: DCN2_OPT_GI_PUSH takes -1, 0 or 1, not %lld",
                        (long long)value);
        g_opt_push.store((int)value, std::memory_order_relaxed);
        return DCN2_OK;
    default:
        return fail(DCN2_EINVAL, "dcn2_set_option: unknown option %d", option);
    }
}

int64_t dcn2_get_option(int option) {
    switch (option) {
    case DCN2_OPT_BWD_SLICE_BYTES: return g_opt_slice_bytes.load(std::memory_order_relaxed);
    case DCN2_OPT_BWD_FUSED: return g_opt_fused.load(std::memory_order_relaxed);
    case DCN2_OPT_GI_PUSH: return g_opt_push.load(std::memory_order_relaxed);
    default: return -2;
    }
}


int dcn2_forward(const dcn2_desc *d, const void *input, const void *weight, const void *mask,
                 const void *offset, const void *bias, void *output, void *workspace,
                 size_t workspace_bytes, void *stream) {
    Geo g;
    int rc = make_geo(d, g);
    if (rc) return rc;
    return forward_impl(g, input, weight, mask, offset, bias, output, workspace, workspace_bytes,
                        stream);
}

int dcn2_backward(const dcn2_desc *d, const void *input, const void *weight, const void *mask,
                  const void *offset, const void *grad_output, void *grad_input,
                  void *grad_offset, void *grad_mask, void *grad_weight, void *grad_bias,
                  void *workspace, size_t workspace_bytes, void *stream) {
    Geo g;
    int rc = make_geo(d, g);
    if (rc) return rc;
    return backward_impl(g, input, weight, mask, offset, grad_output, grad_input, grad_offset,
                         grad_mask, grad_weight, grad_bias, workspace, workspace_bytes, stream);
}

int dcn2_forward_om(const dcn2_desc *d, const void *input, const void *weight, const void *om,
                    const void *bias, void *output, void *workspace, size_t workspace_bytes,
                    void *stream) {
    Geo g;
    long long moff = 0;
    int rc = make_geo(d, g);
    if (rc || (rc = use_om_layout(g, moff))) return rc;
    if (g.B > 0 && !om) return fail(DCN2_EINVAL, "dcn2_forward_om: null om pointer");
    const void *mask = om ? (const char *)om + moff * g.esz : nullptr;
    return forward_impl(g, input, weight, mask, om, bias, output, workspace, workspace_bytes, stream);
}

int dcn2_backward_om(const dcn2_desc *d, const void *input, const void *weight, const void *om,
                     const void *grad_output, void *grad_input, void *grad_om, void *grad_weight,
                     void *grad_bias, void *workspace, size_t workspace_bytes, void *stream) {
    Geo g;
    long long moff = 0;
    int rc = make_geo(d, g);
    if (rc || (rc = use_om_layout(g, moff))) return rc;
    if (g.B > 0 && (!om || !grad_om))
        return fail(DCN2_EINVAL, "dcn2_backward_om: null om/grad_om pointer");
    // with B == 0 the buffers may be NULL; the mask pointers then stay NULL together
    const void *mask = om ? (const char *)om + moff * g.esz : nullptr;
    void *grad_mask = grad_om ? (char *)grad_om + moff * g.esz : nullptr;
    if ((mask == nullptr) != (grad_mask == nullptr))
        return fail(DCN2_EINVAL, "dcn2_backward_om: om and grad_om must both be given");
    return backward_impl(g, input, weight, mask, om, grad_output, grad_input, grad_om, grad_mask,
                         grad_weight, grad_bias, workspace, workspace_bytes, stream);
}

const char *dcn2_last_error(void) { return g_last_error.c_str(); }

#define DCN2_STR_(x) #x
#define DCN2_STR(x) DCN2_STR_(x)
const char *dcn2_version(void) { return "dcnv2_amd " DCN2_STR(DCN2_ABI_VERSION) " gfx950"; }

}  // extern "C"
