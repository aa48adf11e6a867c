// Host-side launchers of the gfx950 kernels.  Each returns hipSuccess or the
// launch error; none synchronises.  Geometry is validated by dcn2_api.cpp
// before any launcher runs.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

struct dcn2_desc;  // include/dcnv2_amd.h

namespace dcn2 {

// Validated problem geometry plus the derived packing sizes.
struct Geo {
    int B, C, H, W, Cout, kh, kw, sh, sw, ph, pw, dh, dw, G;
    int dtype;      // enum dcn2_dtype
    int esz;        // element size in bytes
    int Cg;         // channels per deformable group
    int WG, Cw;     // weight groups and input channels per weight group (C / WG)
    int nhwc;       // input / grad_input are channels-last [B][H][W][C]
    int out_nhwc;   // output / grad_output are channels-last [B][Ho][Wo][Cout]
    int xt_direct;  // nhwc and cs == C: the input itself serves as xt (no repacking)
    int KC;         // channel chunk of one LDS stage (64 for f16/bf16, 32 for f32)
    int Cgp;        // Cg rounded up to KC
    int cs;         // channels-last pixel stride of xt: G*Cgp
    int Ho, Wo, N;  // output spatial size, N = Ho*Wo
    int KK;         // kh*kw
    int Kp;         // packed GEMM K = KK*G*Cgp
    int BM;         // forward block tile in M (128 or 256)
    int Mp;         // Cout rounded up to BM
    // Chunks per tap of the packed K order (G * Cgp / KC), and the weight-group
    // walk: gsplit when every chunk lies in one weight group, group w's chunks
    // of a tap are [w*cpw, (w+1)*cpw) and each group's Cout/WG rows are a
    // multiple of 128, so the GEMMs can run per group over its own chunks.
    int cpt, cpw, gsplit;
    // Offset / mask buffers (and their gradients): elements between images,
    // and whether the mask buffer holds logits that the kernels pass through
    // sigmoid (the offset-and-mask predictor's raw output, dcn2_*_om).
    long long off_bs, msk_bs;
    int msk_logit;
    // The forward runs dcn2_fwd_rw_kernel (weight resident in registers)
    // instead of the chunk-streaming kernels.
    int rw;
    // Process-wide options read once per call (dcn2_set_option): backward
    // slice budget in bytes, fused backward allowed (-1 auto, 0 never),
    // grad_input by cells (-1 auto, 0 per pixel, 1 by cells).
    long long slice_bytes;
    int opt_fused, opt_push;
    // The images of one backward slice (B when the batch runs in one piece).
    int Bs;
};

// dcn2_api.cpp: the descriptor check shared by every entry point, the forward
// on a given workspace, and the per-thread error message (printf-style; returns
// `code`).
int make_geo(const ::dcn2_desc *d, Geo &g);
int forward_impl(const Geo &g, const void *input, const void *weight, const void *mask,
                 const void *offset, const void *bias, void *output, void *workspace,
                 size_t workspace_bytes, void *stream);
int fail(int code, const char *fmt, ...);

// Workspace carving shared by forward and backward (byte offsets).
struct FwdWorkspace {
    size_t xt, wp, tab, total;
};
FwdWorkspace fwd_workspace(const Geo &g);

struct BwdWorkspace {
    size_t xt, wt, tab, gi_acc, gw_acc, gb_acc, cgm, rsc, csum, rec, bcnt, bstart, bcur, sidx, ring, total;
};
// Carves the backward workspace of one slice of g.Bs images.
// Border-ring pixels of one grad_input gather window (4 x the cell tile side).
constexpr int kGatherRing = 64;
BwdWorkspace bwd_workspace(const Geo &g);

// Bucket geometry of the grad_input gather (dcn2_backward.hip): cell tiles
// per row / column, buckets, rows of all buckets together (one per sample),
// bytes per row element, and the bytes of one gather batch's rows with the
// limit they must stay below.
struct GatherGeo {
    int ntx, nty, row_esz;
    int row_scaled;  // bf16 rows carry one scale byte per 32 channels
    long nbuckets, rows;
    long batch_bytes, max_batch_bytes;
    // grad_input by cells (dcn2_gi_push_kernel) or by pixels
    // (dcn2_gi_gather_kernel, which keeps the partial sums of a bucket of
    // several record batches in an fp32 accumulator, gi_acc); both write the
    // caller's grad_input directly
    bool by_cells;
    // bytes of gi_acc (by pixels): one slot of interior pixels per bucket of
    // several record batches, at most rows / (batch + 1) of them
    long acc_bytes;
};
GatherGeo gather_geometry(const Geo &g);

// dcn2_pack.hip: input -> xt (skipped when input is null) and weight -> wp +
// chunk table (skipped when weight is null) in one launch; transpose selects the backward's W'^T fragment
// order.  The input is NCHW, or channels-last when g.nhwc.
// Up to kClearBufs fp32 buffers the pack launch also zeroes (extra workgroups), so
// the backward's accumulators need no launch of their own; n = 0 skips one.
constexpr int kClearBufs = 4;
struct ClearList {
    float *p[kClearBufs];
    size_t n[kClearBufs];
};
hipError_t launch_pack(const Geo &g, const void *input, void *xt, const void *weight, void *wp,
                       void *tab, bool transpose, hipStream_t s, const ClearList *clear = nullptr);

// dcn2_forward.hip
hipError_t launch_forward(const Geo &g, const void *xt, const void *wp, const void *tab,
                          const void *offset, const void *mask, const void *bias, void *out,
                          hipStream_t s);

// dcn2_forward_rw.hip: the resident-weight forward and its eligibility (f16,
// one deformable group of <= 64 channels, 3x3, 128 < Cout <= 256, no weight
// groups).
bool rw_eligible(const Geo &g);
hipError_t launch_forward_rw(const Geo &g, const void *xt, const void *wp, const void *offset,
                             const void *mask, const void *bias, void *out, hipStream_t s);

// dcn2_backward.hip: the backward of g.B images (one slice of the batch; the
// pointers point at its first image).  grad_weight / grad_bias accumulate in
// gw_acc / gb_acc over the slices and are written out when `last` is set.
hipError_t launch_backward(const Geo &g, const void *xt, const void *wt, const void *tab,
                           const void *offset,
                           const void *mask, const void *grad_out, void *grad_input,
                           void *grad_offset, void *grad_mask, void *grad_weight, void *grad_bias,
                           float *gi_acc, float *gw_acc, float *gb_acc, void *cgm, void *rsc,
                           float *csum, void *rec, int *bcnt, int *bstart, int *bcur, int *sidx,
                           float *ring, bool last, hipStream_t s);
// Whether the fused backward kernel may serve g (2-byte type, Cout <= 256),
// and whether it then needs the corner-sum buffer (several chunks per group).
bool fused_bwd_shape(const Geo &g);

}  // namespace dcn2
