/*
 * dcnv2_amd -- C ABI of the MI355X (gfx950) modulated deformable convolution v2.
 *
 * This is the drop-in boundary for the reference's native operator module
 * `Conv2d._C` (reference ext.cpp:15-18, name.h:15-36).  Every entry point takes
 * plain pointers, sizes and a HIP stream handle; there are no framework types.
 * All work is enqueued asynchronously on `stream` (a hipStream_t; NULL = the
 * null stream) and nothing synchronises the host.  The library keeps no state
 * between calls apart from the per-thread error message and the process-wide
 * options of dcn2_set_option, so calls are re-entrant.
 *
 * Semantics are those of torchvision.ops.deform_conv2d(input, offset, weight,
 * bias, stride, padding, dilation, mask), the comparator the reference names:
 *   output[b, m, oy, ox] = bias[m] + sum_{c in group(m), i, j} weight[m, c - c0(m), i, j]
 *                          * mask[b, g*kh*kw + k, oy, ox]
 *                          * bilinear(input[b, c], y, x)
 *   k = i*kw + j,  g = c / (C / deformable_groups),
 *   group(m) = [c0(m), c0(m) + C/weight_groups),  c0(m) = (m / (Cout/weight_groups)) * C/weight_groups,
 *   y = oy*stride_h - pad_h + i*dilation_h + offset[b, 2*(g*kh*kw + k),     oy, ox]
 *   x = ox*stride_w - pad_w + j*dilation_w + offset[b, 2*(g*kh*kw + k) + 1, oy, ox]
 * with bilinear() reading 0 outside the image (reference com.cu:119-148, 187).
 *
 * Tensor layouts are contiguous NCHW in the caller's dtype (input, grad_input,
 * output and grad_output may instead be channels_last, see dcn2_layout):
 *   input  [B, C, H, W]            weight [Cout, C/weight_groups, kh, kw]    bias [Cout]
 *   offset [B, 2*G*kh*kw, Ho, Wo]  mask   [B, G*kh*kw, Ho, Wo]    output [B, Cout, Ho, Wo]
 *   Ho = (H + 2*pad_h - (dilation_h*(kh-1) + 1)) / stride_h + 1   (likewise Wo)
 * All tensors of one call share the dtype in dcn2_desc.dtype.  Every GEMM
 * takes its operands in that dtype and accumulates in fp32 (the sampled
 * columns are rounded to it once, as com.cu:83, 87 rounds them to half); the
 * bilinear sampling arithmetic is fp32.  Intermediate roundings of the
 * backward: the column gradient handed to the grad_input pass is rounded to
 * fp16 (fp16 calls) or to fp16 with one power-of-two scale per 32 channels
 * (bf16 calls: an 11-bit significand over bf16's exponent range); for fp16
 * the one multiplied into the corner sums of grad_offset / grad_mask is
 * rounded to fp16 too (products and sums stay fp32); fp32 has none.
 *
 * Return value of every int function: 0 = success, otherwise a DCN2_E* code;
 * dcn2_last_error() then describes the failure.  This replaces the reference's
 * AT_ASSERTM / std::runtime_error paths (com.cu:209-213, 266-270, 760-761),
 * which the Python layer turns back into RuntimeError.
 */
#ifndef DCNV2_AMD_H
#define DCNV2_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DCN2_ABI_VERSION 4
#define DCN2_API __attribute__((visibility("default")))

enum dcn2_dtype { DCN2_F32 = 0, DCN2_F16 = 1, DCN2_BF16 = 2 };

/* Memory layout of an activation tensor.  DCN2_NHWC is torch's channels_last:
 * [B][H][W][C] (for the output [B][Ho][Wo][Cout]).  dcn2_desc.input_layout
 * covers `input` and `grad_input`: when C/deformable_groups is a multiple of
 * 64 (fp16/bf16) or 32 (fp32) the kernels read such an input in place (it
 * must then be 16-byte aligned) and the forward workspace holds no repacked
 * copy; otherwise it is repacked like an NCHW input.
 * dcn2_desc.output_layout covers `output` (written by the forward) and
 * `grad_output` (read by the backward), both read and written in place.  No
 * counterpart in the reference, which takes and returns contiguous NCHW only. */
enum dcn2_layout { DCN2_NCHW = 0, DCN2_NHWC = 1 };

/* Status codes.  DCN2_ERANGE: the kernels index within one image with 32-bit
 * offsets (the image's base is 64-bit), so per image every tensor must hold
 * fewer than 2^31 elements, the batch at most 65535 images, H and W at most
 * 32767, and the input's channels-last copy must stay below 4 GiB in bytes:
 * (H*W + 1) * G * Cgp * sizeof(dtype) + 256 < 2^32, where Cgp is
 * C/deformable_groups rounded up to 64 (fp16/bf16) or 32 (fp32) channels
 * (e.g. fp32, C = 256, 2048 x 2048 is rejected). */
enum dcn2_status {
    DCN2_OK = 0,
    DCN2_EINVAL = 1,     /* bad geometry, dtype, null pointer or group split     */
    DCN2_EWORKSPACE = 2, /* workspace smaller than dcn2_*_workspace_bytes()       */
    DCN2_ELAUNCH = 3,    /* a HIP launch or runtime call failed                   */
    DCN2_ERANGE = 4      /* a tensor exceeds the library's 32-bit index range     */
};

/* Problem description.  Mirrors the argument list of the reference's
 * dcn_v2_forward(input, weight, mask, offset, bias, stride_h, stride_w, pad_h,
 * pad_w) (name.h:15-24) with the shapes read off the tensors, extended by
 * dilation and deformable groups, which the reference's Python module accepts
 * but never forwards (dcn_v2_mm.py:67-68, 94-102), and by torchvision's weight
 * groups (its deform_conv2d infers them from weight.shape[1]; the reference has
 * none).  weight_groups 0 means 1, so a zero-initialised descriptor is
 * ungrouped; in_channels and out_channels must both divide by it.
 * input_layout and output_layout are enum dcn2_layout values (0 = NCHW). */
typedef struct dcn2_desc {
    int32_t batch, in_channels, height, width;
    int32_t out_channels, kernel_h, kernel_w;
    int32_t stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w;
    int32_t deformable_groups;
    int32_t dtype; /* enum dcn2_dtype */
    int32_t weight_groups;
    int32_t input_layout;
    int32_t output_layout;
} dcn2_desc;

/* Output spatial size for `d`; DCN2_EINVAL if it would be empty. */
DCN2_API int dcn2_output_shape(const dcn2_desc *d, int32_t *out_h, int32_t *out_w);

/* Device workspace the forward / backward need (bytes, 256-byte aligned
 * start required).  0 is returned for an invalid description. */
DCN2_API size_t dcn2_forward_workspace_bytes(const dcn2_desc *d);
DCN2_API size_t dcn2_backward_workspace_bytes(const dcn2_desc *d);

/* Process-wide options (no counterpart in the reference, whose backward holds
 * one image's columns, com.cu:766, and has one code path).  A call reads them
 * once when it starts; set them between calls (a call on another thread that
 * is already running keeps what it read).  The workspace size a call needs
 * depends on them: query dcn2_backward_workspace_bytes after changing one.
 *   DCN2_OPT_BWD_SLICE_BYTES  The backward runs the batch in slices of whole
 *       images, as many per slice as keep its workspace within this many
 *       bytes (at least one image; the slices are made equal in size up to
 *       one image).  Default DCN2_BWD_SLICE_BYTES_DEFAULT; minimum 1.
 *   DCN2_OPT_BWD_FUSED  -1 (default): the backward uses its fused
 *       column-gradient + grad_weight kernel where the shape allows it;
 *       0: never (two kernels).
 *   DCN2_OPT_GI_PUSH  -1 (default): grad_input by cells where the buckets
 *       are dense enough, per pixel otherwise; 1: by cells; 0: per pixel.
 * dcn2_set_option returns DCN2_EINVAL for an unknown option or value;
 * dcn2_get_option returns the current value (-2 for an unknown option). */
enum dcn2_option { DCN2_OPT_BWD_SLICE_BYTES = 0, DCN2_OPT_BWD_FUSED = 1, DCN2_OPT_GI_PUSH = 2 };
#define DCN2_BWD_SLICE_BYTES_DEFAULT ((int64_t)192 << 20)
DCN2_API int dcn2_set_option(int option, int64_t value);
DCN2_API int64_t dcn2_get_option(int option);

/* Forward.  Replaces MyDCN_forward / _C.dcn_v2_forward (com.cu:198-272,
 * ext.cpp:16; bound in dcn_v2_mm.py:20-30).  `mask` may be NULL (all ones,
 * DCNv1) and `bias` may be NULL (zeros).  `output` is fully overwritten. */
DCN2_API int dcn2_forward(const dcn2_desc *d, const void *input, const void *weight, const void *mask,
                 const void *offset, const void *bias, void *output, void *workspace,
                 size_t workspace_bytes, void *stream);

/* Backward.  Replaces MyDCN_backward / _C.dcn_v2_backward (com.cu:733-848,
 * ext.cpp:17; bound in dcn_v2_mm.py:38-49), whose result order is
 * [grad_input, grad_offset, grad_mask, grad_weight, grad_bias] (com.cu:845-847).
 * All five gradient buffers are fully overwritten (not accumulated).
 * grad_mask must be NULL exactly when mask is NULL; grad_bias may be NULL. */
DCN2_API int dcn2_backward(const dcn2_desc *d, const void *input, const void *weight, const void *mask,
                  const void *offset, const void *grad_output, void *grad_input,
                  void *grad_offset, void *grad_mask, void *grad_weight, void *grad_bias,
                  void *workspace, size_t workspace_bytes, void *stream);

/* Forward and backward on the offset-and-mask predictor's raw output.  No
 * counterpart in the reference's C++: they replace the chunk(3) / cat / sigmoid
 * its DCN module applies to conv_offset_mask(x) before calling the operator
 * (dcn_v2_mm.py:133-137), so the kernels read that tensor directly.
 *   om      [B, 3*G*kh*kw, Ho, Wo]: channels [0, 2*G*kh*kw) are the offsets,
 *           in the layout of dcn2_forward's `offset`; channels
 *           [2*G*kh*kw, 3*G*kh*kw) are mask logits, mask = sigmoid(logit)
 *           (computed in fp32 from the stored value).
 *   grad_om same shape: the offset gradient in the first 2*G*kh*kw channels,
 *           the gradient of the logits, grad_mask * mask * (1 - mask), in the
 *           rest; fully overwritten.
 * Everything else (including the workspace, sized by
 * dcn2_forward_workspace_bytes / dcn2_backward_workspace_bytes of the same
 * descriptor) is as in dcn2_forward / dcn2_backward. */
DCN2_API int dcn2_forward_om(const dcn2_desc *d, const void *input, const void *weight, const void *om,
                    const void *bias, void *output, void *workspace, size_t workspace_bytes,
                    void *stream);
DCN2_API int dcn2_backward_om(const dcn2_desc *d, const void *input, const void *weight, const void *om,
                     const void *grad_output, void *grad_input, void *grad_om, void *grad_weight,
                     void *grad_bias, void *workspace, size_t workspace_bytes, void *stream);

/* Forward without allocation or workspace.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Arguments
 * and results are those of dcn2_forward; the workspace is a static device
 * array of DCN2_NOALLOC_SCRATCH_BYTES that the library holds on every GPU it
 * runs on until the process ends (its address is looked up once per device on
 * the first call there).  A problem whose dcn2_forward_workspace_bytes()
 * exceeds that size is rejected with DCN2_EWORKSPACE before anything is
 * launched.  Every call on one GPU uses the same array: calls that overlap on
 * one GPU (concurrent streams or threads) race and must be serialised by the
 * caller; consecutive calls on one stream are safe.  Nothing is allocated and
 * nothing synchronises.  Under HIP graph capture: make the first call on a
 * device before capturing (it looks the array up with hipGetSymbolAddress);
 * later calls capture as kernel nodes only (no memset, no allocation). */
#define DCN2_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
DCN2_API int dcn2_forward_noalloc(const dcn2_desc *d, const void *input, const void *weight,
                                  const void *mask, const void *offset, const void *bias,
                                  void *output, void *stream);

/* Per-stage kernel timing (no counterpart in the reference, whose timing loops
 * live inside its forward, com_2buffer_cpasyc.cu:334-392).  While enabled on
 * the calling thread, every stage of dcn2_forward / dcn2_backward is bracketed
 * by HIP events recorded on the call's stream; dcn2_profile_read() waits for
 * the recorded events, returns the summed milliseconds and launch count of
 * one stage, and clears that stage.  Disabled by default; enabling adds two
 * event records per stage and nothing else. */
enum dcn2_stage {
    DCN2_STAGE_FWD_PACK = 0,     /* input / weight repacking of the forward      */
    DCN2_STAGE_FWD_MAIN = 1,     /* fused sampling + MFMA forward kernel          */
    DCN2_STAGE_BWD_PACK = 2,     /* repacking and accumulator clearing            */
    DCN2_STAGE_BWD_COLGRAD = 3,  /* column gradient, grad_offset, grad_mask; with
                                    the fused backward kernel also grad_weight /
                                    grad_bias (DCN2_STAGE_BWD_GRADW then records
                                    no launch)                                   */
    DCN2_STAGE_BWD_GRADW = 4,    /* grad_weight / grad_bias                        */
    DCN2_STAGE_BWD_GATHER = 5,   /* grad_input; by cells (dense buckets) it is
                                    written in the caller's dtype and layout here,
                                    grad_weight / grad_bias finalised with it     */
    DCN2_STAGE_BWD_FINAL = 6,    /* conversion to the caller's dtype and layout
                                    (per-pixel grad_input only)                  */
    DCN2_STAGE_BWD_BUCKET = 7,   /* grad_input bucket passes (count, scan + place) */
    DCN2_STAGE_COUNT = 8
};
DCN2_API int dcn2_profile_enable(int on);
DCN2_API int dcn2_profile_read(int stage, double *total_ms, int *launches);

/* Human-readable description of the last failure on the calling thread. */
DCN2_API const char *dcn2_last_error(void);

/* Library version string ("dcnv2_amd <abi> gfx950"). */
DCN2_API const char *dcn2_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DCNV2_AMD_H */
