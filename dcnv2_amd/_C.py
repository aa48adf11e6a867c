"""Native operator module: the drop-in for the reference's ``Conv2d._C``.

The reference builds ``Conv2d._C`` as a pybind11 extension exporting
``dcn_v2_forward`` and ``dcn_v2_backward`` (reference ``ext.cpp:15-18``,
``name.h:15-36``).  Here the same two functions, with the same positional
arguments and result order, bind the C ABI of ``lib/libdcnv2_amd.so``
(``include/dcnv2_amd.h``) through ctypes.  Torch supplies only device memory
(outputs and the scratch workspace come from its caching allocator, as the
reference's ``at::zeros``/``at::empty`` do, ``com.cu:232-235, 766-774``) and
the current stream; all arithmetic runs in the gfx950 kernels of the library.

Extensions over the reference, all trailing and optional: ``dilation_h``,
``dilation_w`` and ``deformable_groups`` (the reference's Python module accepts
them but never forwards them, ``dcn_v2_mm.py:67-68, 94-102``); fp16/bf16 as
well as fp32 tensors; ``mask`` and ``bias`` may be ``None``; a weight of shape
``[Cout, C/groups, kh, kw]`` selects torchvision's weight groups; a
``channels_last`` input is read without a layout copy, its output and
``grad_input`` come back channels_last (as torch's own convolutions propagate
the memory format), and a ``channels_last`` ``grad_output`` is read in place.

Errors: any invalid device, dtype, shape or launch failure raises
``RuntimeError``, as the reference's ``AT_ASSERTM`` checks do
(``com.cu:209-213, 743-747, 760-761``).  There is no CPU fallback: without the
built library every call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libdcnv2_amd.so")
_DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
_lib = None
_lib_lock = threading.Lock()


class Desc(ctypes.Structure):
    """``dcn2_desc`` of ``include/dcnv2_amd.h``."""
    _fields_ = [(name, ctypes.c_int32) for name in (
        "batch", "in_channels", "height", "width", "out_channels", "kernel_h", "kernel_w",
        "stride_h", "stride_w", "pad_h", "pad_w", "dilation_h", "dilation_w",
        "deformable_groups", "dtype", "weight_groups", "input_layout", "output_layout")]


def library_path() -> str:
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    """Loads libdcnv2_amd.so once; raises RuntimeError if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise RuntimeError(
                    f"dcnv2_amd: native library {_LIB_PATH} is not built; "
                    "run `python -m dcnv2_amd.build` (or __graft_entry__.build())")
            L = ctypes.CDLL(_LIB_PATH)
            vp, sz, dp = ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(Desc)
            L.dcn2_output_shape.argtypes = [dp, ctypes.POINTER(ctypes.c_int32),
                                            ctypes.POINTER(ctypes.c_int32)]
            L.dcn2_output_shape.restype = ctypes.c_int
            L.dcn2_forward_workspace_bytes.argtypes = [dp]
            L.dcn2_forward_workspace_bytes.restype = sz
            L.dcn2_backward_workspace_bytes.argtypes = [dp]
            L.dcn2_backward_workspace_bytes.restype = sz
            L.dcn2_forward.argtypes = [dp] + [vp] * 7 + [sz, vp]
            L.dcn2_forward.restype = ctypes.c_int
            L.dcn2_backward.argtypes = [dp] + [vp] * 11 + [sz, vp]
            L.dcn2_backward.restype = ctypes.c_int
            L.dcn2_forward_om.argtypes = [dp] + [vp] * 6 + [sz, vp]
            L.dcn2_forward_om.restype = ctypes.c_int
            L.dcn2_backward_om.argtypes = [dp] + [vp] * 9 + [sz, vp]
            L.dcn2_backward_om.restype = ctypes.c_int
            L.dcn2_forward_noalloc.argtypes = [dp] + [vp] * 7
            L.dcn2_forward_noalloc.restype = ctypes.c_int
            L.dcn2_last_error.argtypes = []
            L.dcn2_last_error.restype = ctypes.c_char_p
            L.dcn2_version.argtypes = []
            L.dcn2_version.restype = ctypes.c_char_p
            L.dcn2_profile_enable.argtypes = [ctypes.c_int]
            L.dcn2_profile_enable.restype = ctypes.c_int
            L.dcn2_profile_read.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                            ctypes.POINTER(ctypes.c_int)]
            L.dcn2_profile_read.restype = ctypes.c_int
            L.dcn2_set_option.argtypes = [ctypes.c_int, ctypes.c_int64]
            L.dcn2_set_option.restype = ctypes.c_int
            L.dcn2_get_option.argtypes = [ctypes.c_int]
            L.dcn2_get_option.restype = ctypes.c_int64
            _lib = L
    return _lib


def _err(prefix: str) -> RuntimeError:
    return RuntimeError(f"{prefix}: {lib().dcn2_last_error().decode()}")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _layout(t):
    """(t, layout): a channels_last activation (one that is not also contiguous
    NCHW) is handed over as it is, with layout 1 (``DCN2_NHWC``); anything
    else becomes contiguous NCHW, layout 0.  The kernels read a channels_last
    input in place when its channels need no padding, and a channels_last
    grad_output always."""
    cl = torch.channels_last
    if t.dim() == 4 and not t.is_contiguous() and t.is_contiguous(memory_format=cl):
        if t.data_ptr() % 16:  # in-place reads use 16-byte loads
            t = t.clone(memory_format=cl)
        return t, 1
    return t.contiguous(), 0


_input_layout = _layout


def make_desc(input, weight, stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w,
              deformable_groups, input_layout=0, output_layout=0) -> Desc:
    B, C, H, W = (int(v) for v in input.shape)
    Cout, Cw, kh, kw = (int(v) for v in weight.shape)
    # weight groups follow from weight.shape[1], as in torchvision's deform_conv2d
    return Desc(B, C, H, W, Cout, kh, kw, int(stride_h), int(stride_w), int(pad_h), int(pad_w),
                int(dilation_h), int(dilation_w), int(deformable_groups), _DTYPES[input.dtype],
                C // Cw, int(input_layout), int(output_layout))


def _empty_out(shape, like, layout):
    """The output tensor: channels_last when `layout` is 1."""
    fmt = torch.channels_last if layout else torch.contiguous_format
    return torch.empty(shape, dtype=like.dtype, device=like.device, memory_format=fmt)


def _validate(name, input, weight, mask, offset, bias, extra=()):
    tensors = {"input": input, "weight": weight, "offset": offset}
    if mask is not None:
        tensors["mask"] = mask
    if bias is not None:
        tensors["bias"] = bias
    tensors.update(dict(extra))
    for k, t in tensors.items():
        if not isinstance(t, torch.Tensor):
            raise RuntimeError(f"{name}: {k} must be a tensor")
        if not t.is_cuda:  # reference com.cu:209-213
            raise RuntimeError(f"{name}: {k} must be a GPU (HIP) tensor")
    dev = input.device
    for k, t in tensors.items():
        if t.device != dev:
            raise RuntimeError(f"{name}: {k} is on {t.device}, input on {dev}")
        if t.dtype != input.dtype:
            raise RuntimeError(f"{name}: {k} has dtype {t.dtype}, input has {input.dtype}")
    if input.dtype not in _DTYPES:
        raise RuntimeError(f"{name}: unsupported dtype {input.dtype} "
                           "(float32, float16 and bfloat16 are supported)")
    if input.dim() != 4 or weight.dim() != 4 or offset.dim() != 4:
        raise RuntimeError(f"{name}: input, weight and offset must be 4-D")
    # reference com.cu:760-761 requires weight.shape[1] == C; torchvision's weight
    # groups (C / weight.shape[1] of them) must also split Cout evenly
    C, Cw, Cout = int(input.shape[1]), int(weight.shape[1]), int(weight.shape[0])
    if Cw <= 0 or C % Cw != 0 or Cout % (C // Cw) != 0:
        raise RuntimeError(f"{name}: input has {C} channels, weight expects {Cw} per group "
                           f"with {Cout} output channels")
    if bias is not None and tuple(bias.shape) != (weight.shape[0],):
        raise RuntimeError(f"{name}: bias shape {tuple(bias.shape)} != ({weight.shape[0]},)")


def _geometry(name, desc, input, mask, offset):
    ho, wo = ctypes.c_int32(), ctypes.c_int32()
    if lib().dcn2_output_shape(ctypes.byref(desc), ctypes.byref(ho), ctypes.byref(wo)) != 0:
        raise _err(name)
    B, G, KK = desc.batch, desc.deformable_groups, desc.kernel_h * desc.kernel_w
    want_off = (B, 2 * G * KK, ho.value, wo.value)
    if tuple(offset.shape) != want_off:
        raise RuntimeError(f"{name}: offset shape {tuple(offset.shape)} != {want_off}")
    if mask is not None and tuple(mask.shape) != (B, G * KK, ho.value, wo.value):
        raise RuntimeError(f"{name}: mask shape {tuple(mask.shape)} != "
                           f"{(B, G * KK, ho.value, wo.value)}")
    return ho.value, wo.value


def _workspace(nbytes, device):
    # 256 extra bytes so the start can be aligned to 256 whatever the allocator returns
    buf = torch.empty(int(nbytes) + 256, dtype=torch.uint8, device=device)
    addr = buf.data_ptr()
    aligned = (addr + 255) & ~255
    return buf, aligned, int(nbytes)


def dcn_v2_forward(input, weight, mask, offset, bias, stride_h, stride_w, pad_h, pad_w,
                   dilation_h=1, dilation_w=1, deformable_groups=1):
    """Reference ``MyDCN_forward`` (``com.cu:198-272``): returns the output
    ``[B, Cout, Ho, Wo]`` in the input dtype."""
    name = "dcn_v2_forward"
    _validate(name, input, weight, mask, offset, bias)
    input, layout = _input_layout(input)
    weight, offset = weight.contiguous(), offset.contiguous()
    mask = mask.contiguous() if mask is not None else None
    bias = bias.contiguous() if bias is not None else None
    desc = make_desc(input, weight, stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w,
                     deformable_groups, layout, layout)
    ho, wo = _geometry(name, desc, input, mask, offset)
    L = lib()
    out = _empty_out((desc.batch, desc.out_channels, ho, wo), input, layout)
    with torch.cuda.device(input.device):
        ws_buf, ws, ws_bytes = _workspace(L.dcn2_forward_workspace_bytes(ctypes.byref(desc)),
                                          input.device)
        stream = torch.cuda.current_stream(input.device).cuda_stream
        rc = L.dcn2_forward(ctypes.byref(desc), _ptr(input), _ptr(weight), _ptr(mask),
                            _ptr(offset), _ptr(bias), _ptr(out), ctypes.c_void_p(ws), ws_bytes,
                            ctypes.c_void_p(stream))
    if rc != 0:
        raise _err(name)
    del ws_buf  # returned to torch's caching allocator in stream order
    return out


def dcn_v2_backward(input, weight, mask, offset, bias, grad_output, stride_h, stride_w, pad_h,
                    pad_w, dilation_h=1, dilation_w=1, deformable_groups=1):
    """Reference ``MyDCN_backward`` (``com.cu:733-848``): returns
    ``[grad_input, grad_offset, grad_mask, grad_weight, grad_bias]`` (the order
    of ``com.cu:845-847``); ``grad_mask``/``grad_bias`` are ``None`` when
    ``mask``/``bias`` is."""
    name = "dcn_v2_backward"
    _validate(name, input, weight, mask, offset, bias, extra=[("grad_output", grad_output)])
    input, layout = _input_layout(input)
    weight, offset = weight.contiguous(), offset.contiguous()
    mask = mask.contiguous() if mask is not None else None
    grad_output, go_layout = _layout(grad_output)
    desc = make_desc(input, weight, stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w,
                     deformable_groups, layout, go_layout)
    ho, wo = _geometry(name, desc, input, mask, offset)
    if tuple(grad_output.shape) != (desc.batch, desc.out_channels, ho, wo):
        raise RuntimeError(f"{name}: grad_output shape {tuple(grad_output.shape)} != "
                           f"{(desc.batch, desc.out_channels, ho, wo)}")
    L = lib()
    grad_input = torch.empty_like(input)  # keeps the channels_last layout of layout 1
    grad_offset = torch.empty_like(offset)
    grad_mask = torch.empty_like(mask) if mask is not None else None
    grad_weight = torch.empty_like(weight)
    grad_bias = torch.empty((desc.out_channels,), dtype=input.dtype, device=input.device) \
        if bias is not None else None
    with torch.cuda.device(input.device):
        ws_buf, ws, ws_bytes = _workspace(L.dcn2_backward_workspace_bytes(ctypes.byref(desc)),
                                          input.device)
        stream = torch.cuda.current_stream(input.device).cuda_stream
        rc = L.dcn2_backward(ctypes.byref(desc), _ptr(input), _ptr(weight), _ptr(mask),
                             _ptr(offset), _ptr(grad_output), _ptr(grad_input),
                             _ptr(grad_offset), _ptr(grad_mask), _ptr(grad_weight),
                             _ptr(grad_bias), ctypes.c_void_p(ws), ws_bytes,
                             ctypes.c_void_p(stream))
    if rc != 0:
        raise _err(name)
    del ws_buf
    return [grad_input, grad_offset, grad_mask, grad_weight, grad_bias]


def _om_geometry(name, desc, om):
    ho, wo = ctypes.c_int32(), ctypes.c_int32()
    if lib().dcn2_output_shape(ctypes.byref(desc), ctypes.byref(ho), ctypes.byref(wo)) != 0:
        raise _err(name)
    want = (desc.batch, 3 * desc.deformable_groups * desc.kernel_h * desc.kernel_w, ho.value,
            wo.value)
    if tuple(om.shape) != want:
        raise RuntimeError(f"{name}: om shape {tuple(om.shape)} != {want}")
    return ho.value, wo.value


def dcn_v2_forward_om(input, weight, om, bias, stride_h, stride_w, pad_h, pad_w,
                      dilation_h=1, dilation_w=1, deformable_groups=1):
    """Forward on the offset-and-mask predictor's raw output ``om``
    ``[B, 3*G*kh*kw, Ho, Wo]``: offsets are its first ``2*G*kh*kw`` channels and
    the mask is ``sigmoid`` of the rest, exactly the split the reference's
    ``DCN.forward`` makes with ``chunk(3)`` / ``cat`` / ``sigmoid``
    (``dcn_v2_mm.py:133-137``), done inside the kernels."""
    name = "dcn_v2_forward_om"
    _validate(name, input, weight, None, om, bias)
    input, layout = _input_layout(input)
    weight, om = weight.contiguous(), om.contiguous()
    bias = bias.contiguous() if bias is not None else None
    desc = make_desc(input, weight, stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w,
                     deformable_groups, layout, layout)
    ho, wo = _om_geometry(name, desc, om)
    L = lib()
    out = _empty_out((desc.batch, desc.out_channels, ho, wo), input, layout)
    with torch.cuda.device(input.device):
        ws_buf, ws, ws_bytes = _workspace(L.dcn2_forward_workspace_bytes(ctypes.byref(desc)),
                                          input.device)
        stream = torch.cuda.current_stream(input.device).cuda_stream
        rc = L.dcn2_forward_om(ctypes.byref(desc), _ptr(input), _ptr(weight), _ptr(om),
                               _ptr(bias), _ptr(out), ctypes.c_void_p(ws), ws_bytes,
                               ctypes.c_void_p(stream))
    if rc != 0:
        raise _err(name)
    del ws_buf
    return out


def dcn_v2_backward_om(input, weight, om, bias, grad_output, stride_h, stride_w, pad_h, pad_w,
                       dilation_h=1, dilation_w=1, deformable_groups=1):
    """Backward of :func:`dcn_v2_forward_om`: returns ``[grad_input, grad_om,
    grad_weight, grad_bias]``; ``grad_om`` holds the offset gradient and the
    gradient of the mask logits (``grad_mask * mask * (1 - mask)``)."""
    name = "dcn_v2_backward_om"
    _validate(name, input, weight, None, om, bias, extra=[("grad_output", grad_output)])
    input, layout = _input_layout(input)
    weight, om = weight.contiguous(), om.contiguous()
    grad_output, go_layout = _layout(grad_output)
    desc = make_desc(input, weight, stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w,
                     deformable_groups, layout, go_layout)
    ho, wo = _om_geometry(name, desc, om)
    if tuple(grad_output.shape) != (desc.batch, desc.out_channels, ho, wo):
        raise RuntimeError(f"{name}: grad_output shape {tuple(grad_output.shape)} != "
                           f"{(desc.batch, desc.out_channels, ho, wo)}")
    L = lib()
    grad_input = torch.empty_like(input)  # keeps the channels_last layout of layout 1
    grad_om = torch.empty_like(om)
    grad_weight = torch.empty_like(weight)
    grad_bias = torch.empty((desc.out_channels,), dtype=input.dtype, device=input.device) \
        if bias is not None else None
    with torch.cuda.device(input.device):
        ws_buf, ws, ws_bytes = _workspace(L.dcn2_backward_workspace_bytes(ctypes.byref(desc)),
                                          input.device)
        stream = torch.cuda.current_stream(input.device).cuda_stream
        rc = L.dcn2_backward_om(ctypes.byref(desc), _ptr(input), _ptr(weight), _ptr(om),
                                _ptr(grad_output), _ptr(grad_input), _ptr(grad_om),
                                _ptr(grad_weight), _ptr(grad_bias), ctypes.c_void_p(ws),
                                ws_bytes, ctypes.c_void_p(stream))
    if rc != 0:
        raise _err(name)
    del ws_buf
    return [grad_input, grad_om, grad_weight, grad_bias]


def version() -> str:
    return lib().dcn2_version().decode()


# process-wide options of the library (enum dcn2_option)
OPTIONS = ("bwd_slice_bytes", "bwd_fused", "gi_push")


def set_option(name: str, value: int) -> None:
    """bwd_slice_bytes: backward workspace budget per slice of images;
    bwd_fused: -1 automatic, 0 never the fused backward kernel; gi_push: -1
    automatic, 0 per-pixel grad_input, 1 by cells."""
    if lib().dcn2_set_option(OPTIONS.index(name), int(value)) != 0:
        raise _err("set_option")


def get_option(name: str) -> int:
    return int(lib().dcn2_get_option(OPTIONS.index(name)))


class option:
    """Context manager: `with option("gi_push", 0): ...` sets an option and
    restores its previous value on exit."""

    def __init__(self, name: str, value: int):
        self.name, self.value = name, value

    def __enter__(self):
        self.prev = get_option(self.name)
        set_option(self.name, self.value)
        return self

    def __exit__(self, *exc):
        set_option(self.name, self.prev)
        return False


STAGES = ("fwd_pack", "fwd_main", "bwd_pack", "bwd_colgrad", "bwd_gradw", "bwd_gather",
          "bwd_final", "bwd_bucket")


def profile_enable(on: bool = True) -> None:
    """Per-stage HIP-event timing of the calls made on this thread."""
    lib().dcn2_profile_enable(1 if on else 0)


def profile_read(stage: str):
    """(total_ms, launches) recorded for `stage` since the last read; waits for
    the recorded events."""
    ms, n = ctypes.c_double(), ctypes.c_int()
    if lib().dcn2_profile_read(STAGES.index(stage), ctypes.byref(ms), ctypes.byref(n)) != 0:
        raise _err("profile_read")
    return ms.value, n.value
