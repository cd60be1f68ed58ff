"""ctypes binding of libpisa_hip.so (the C ABI declared in include/pisa_hip.h).

Only this module touches raw pointers.  Tensors are described by
``pisa_view`` structs (data pointer + batch/head/token strides, unit head_dim
stride); every call is enqueued on PyTorch's current stream of the tensor's
device, and a non-zero status is raised as ``RuntimeError`` carrying the
library's own message.  Loading fails loudly (``ImportError``) when the shared
library has not been built - there is no fallback implementation.
"""
from __future__ import annotations

import contextlib
import ctypes
import pathlib

import torch  # must be imported first: the library then binds to torch's HIP runtime

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libpisa_hip.so"

DTYPE_BF16 = 0
DTYPE_F16 = 1
DTYPE_F32 = 2
STATS_MEANS = 0
STATS_HYD = 1
STATS_GENERIC = 2
STATS_FLAG_VALUE_SUMS = 0x100
ROUTE_HYD = 0
ROUTE_CENTROID = 1
NO_SINK = -2
MASK_NONE = 0
MASK_BOOL = 1
MASK_ADD_F32 = 2
MASK_ADD_F16 = 3
MASK_ADD_BF16 = 4
NOALLOC_SCRATCH_BYTES = 192 << 20  # static scratch of pisa_hip_forward_noalloc

_DTYPES = {torch.bfloat16: DTYPE_BF16, torch.float16: DTYPE_F16, torch.float32: DTYPE_F32}


class PisaView(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("batch_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64),
        ("token_stride", ctypes.c_int64),
    ]


class PisaMask(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("kind", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("batch_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64),
        ("query_stride", ctypes.c_int64),
        ("key_stride", ctypes.c_int64),
    ]


class PisaTokenGrid(ctypes.Structure):
    _fields_ = [("frames", ctypes.c_int32), ("height", ctypes.c_int32), ("width", ctypes.c_int32)]


_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_vp = ctypes.c_void_p

_SIGNATURES = {
    "pisa_hip_api_version": (ctypes.c_int, []),
    "pisa_hip_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "pisa_hip_last_error": (ctypes.c_char_p, []),
    "pisa_hip_build_info": (ctypes.c_int, [ctypes.c_char_p, _i64]),
    "pisa_hip_forward_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i32]),
    "pisa_hip_forward": (
        ctypes.c_int,
        [_i32, _i32, _i32, _i32, _i32, PisaView, PisaView, PisaView, PisaView, PisaTokenGrid,
         _i32, _f32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _i64, _vp],
    ),
    "pisa_hip_forward_noalloc": (
        ctypes.c_int,
        [_i32, _i32, _i32, _i32, _i32, PisaView, PisaView, PisaView, PisaView, PisaTokenGrid,
         _i32, _f32, _i32, _i32, _i32, _i32, _vp],
    ),
    "pisa_hip_prepare": (
        ctypes.c_int,
        [_i32, _i32, _i32, _i32, _i32, PisaView, PisaView, PisaView, PisaView, PisaTokenGrid,
         _i32, _f32, _i32, _i32, _i32, _i32, _vp, _i64, _vp],
    ),
    "pisa_hip_attend": (
        ctypes.c_int,
        [_i32, _i32, _i32, _i32, _i32, PisaView, PisaView, PisaView, PisaView, PisaTokenGrid,
         _i32, _f32, _i32, _i32, _i32, _i32, _vp, _i64, _vp],
    ),
    "pisa_hip_block_stats_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32]),
    "pisa_hip_block_stats": (
        ctypes.c_int,
        [_i32, _i32, _i32, _i32, _i32, _i32, PisaView, PisaView, PisaView, PisaTokenGrid, _i32,
         _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp],
    ),
    "pisa_hip_route_topk": (
        ctypes.c_int,
        [_i32, _i32, _i32, _vp, _vp, _vp, _i32, _f32, _i32, _i32, _vp, _vp, _vp],
    ),
    "pisa_hip_pack_spatial_qkv": (
        ctypes.c_int,
        [_i32, _i32, _i32, _i32, _i32, PisaView, PisaView, PisaView, PisaTokenGrid, _vp, _vp, _vp, _vp],
    ),
    "pisa_hip_unpack_spatial_output": (
        ctypes.c_int,
        [_i32, _i32, _i32, _i32, _i32, _vp, PisaTokenGrid, _vp, _vp],
    ),
    "pisa_hip_fuse_spatial_epilogue": (
        ctypes.c_int,
        [_i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, PisaTokenGrid, _vp, _vp],
    ),
    "attn_hip_dense_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32]),
    "attn_hip_dense_forward": (
        ctypes.c_int,
        [_i32, _i32, _i32, _i32, _i32, _i32, PisaView, PisaView, PisaView, PisaView, _f32, _vp, _i64, _vp],
    ),
    "attn_hip_fixed_block_forward": (
        ctypes.c_int,
        [_i32, _i32, _i32, _i32, _i32, _i32, PisaView, PisaView, PisaView, PisaView, _f32, _i32, _vp],
    ),
    "attn_hip_fixed_block_forward_masked": (
        ctypes.c_int,
        [_i32, _i32, _i32, _i32, _i32, _i32, PisaView, PisaView, PisaView, PisaView, _f32, _i32, PisaMask, _vp],
    ),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH.name} is not built; run `python __graft_entry__.py` or "
            f"`python comfyui-rdna35-attention_amd/build_lib.py` (hipcc, gfx950)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


LIB = _load()


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError as exc:
        raise ValueError(f"unsupported dtype {dtype}") from exc


def check(status: int, what: str) -> None:
    if status != 0:
        reason = LIB.pisa_hip_status_string(status).decode()
        detail = LIB.pisa_hip_last_error().decode()
        raise RuntimeError(f"{what} failed ({reason}): {detail}")


def view4(tensor: torch.Tensor) -> PisaView:
    """[B, H, T, D] tensor with unit D stride."""
    sb, sh, st, sd = tensor.stride()
    if sd != 1:
        raise ValueError("head_dim must have unit stride")
    return PisaView(tensor.data_ptr(), sb, sh, st)


def view3(tensor: torch.Tensor) -> PisaView:
    """[BH, T, D] tensor with unit D stride (batch=BH, heads=1)."""
    if tensor.stride(2) != 1:
        raise ValueError("head_dim must have unit stride")
    return PisaView(tensor.data_ptr(), tensor.stride(0), 0, tensor.stride(1))


def grid(frames: int = 0, height: int = 0, width: int = 0) -> PisaTokenGrid:
    return PisaTokenGrid(frames, height, width)


# torch's raw current-stream query (what its own compiled kernels launch on);
# the public torch.cuda.current_stream builds a Stream object per call
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """hipStream_t (as an int) of the current stream of `device`."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def on_device(device: torch.device):
    """Device guard around a launch; a no-op when `device` is already the current device."""
    if device.index is None or device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


def build_info_string() -> str:
    buf = ctypes.create_string_buffer(1024)
    check(LIB.pisa_hip_build_info(buf, len(buf)), "pisa_hip_build_info")
    return buf.value.decode()
