"""ctypes binding of libleatmi.so (include/leatmi.h), the gfx950 HIP kernels.

The library links the HIP runtime by its soname, libamdhip64.so.7; torch is imported first so
that the dynamic loader binds it to the runtime torch already loaded, and the two share
devices, streams and memory. There is no fallback: without the built library or a gfx950 GPU
every call raises.
"""

from __future__ import annotations

import ctypes
import functools
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

LIB_PATH = Path(__file__).resolve().parent / "libleatmi.so"

_p, _i, _i64, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float

# name: argument types, as include/leatmi.h declares them
SIGNATURES: dict[str, list] = {
    "leat_quantize_q8": [_p, _i, _i, _p, _f, _p, _p, _p, _p],
    "leat_matvec": [_i, _p, _i, _i, _p, _p, _p, _i, _p, _p, _p],
    "leat_matvecs": [_i, _p, _p, _p, _i, _p, _p, _p, _i, _p, _p],
    "leat_glu_matvec": [_i, _p, _p, _i, _i, _p, _p, _p, _i, _i, _p, _p],
    "leat_matvec_f32x": [_i, _p, _i, _i, _p, _i, _p, _p, _p],
    "leat_dequantize": [_i, _p, _i64, _p, _p],
    "leat_group_dots": [_i, _p, _i, _i, _p, _i, _p, _p],
    "leat_matmul_workspace": [_i, _i, _i, _i, _i],
    "leat_matmul": [_i, _p, _i, _i, _p, _p, _p, _i, _p, _p, _p, _i64, _p],
    "leat_matmul_noalloc": [_i, _p, _i, _i, _p, _p, _p, _i, _p, _p, _p],
    "leat_glu_matmul": [_i, _p, _p, _i, _i, _p, _p, _p, _i, _i, _p, _p, _i64, _p],
    "leat_route": [_p, _i, _i, _i, _p, _p, _p],
    "leat_scores": [_p, _i, _i, _p, _f, _p, _i, _p, _p],
    "leat_experts_glu": [_i, _p, _p, _i, _i, _i, _p, _p, _p, _p, _i, _i, _p, _p, _i, _p, _p],
    "leat_experts_down": [_i, _p, _i, _i, _i, _p, _p, _p, _p, _p, _i, _i, _p, _p, _p, _p, _p],
    "leat_experts_glu_f32": [_i, _p, _p, _i, _i, _i, _p, _i, _p, _f, _p, _i, _p, _p, _i, _p, _p, _p, _p, _p, _p, _p],
    "leat_matvecs_f32": [_i, _p, _p, _p, _i, _p, _i, _p, _f, _p, _p],
    "leat_matvec_f32": [_i, _p, _i, _i, _p, _i, _p, _f, _p, _p, _p],
    "leat_glu_matvec_q8": [_i, _p, _p, _i, _i, _p, _p, _p, _i, _i, _p, _p, _p, _p, _p],
    "leat_glu_matmul_q8": [_i, _p, _p, _i, _i, _p, _p, _p, _i, _i, _p, _p, _p, _p, _p, _i64, _p],
    "leat_embedding": [_i, _p, _i, _i, _p, _i, _p, _p],
    "leat_rotate": [_p, _p, _p, _i, _i, _i, _i, _p, _p, _i, _i, _p, _p, _p, _p, _i, _i, _p],
    "leat_attention_workspace": [_i, _i, _i],
    "leat_qkv_rotate_f32": [_i, _p, _p, _p, _i, _i, _i, _i, _p, _i, _p, _f, _p, _p, _i, _p, _p, _p, _p, _i, _i, _p],
    "leat_attention": [_p, _p, _i, _i, _i, _i, _i, _i, _p, _p, _i, _f, _p, _i64, _p, _p],
    "leat_attention_q8": [_p, _p, _i, _i, _i, _i, _i, _i, _p, _p, _i, _f, _p, _i64, _p, _p, _p, _p, _p],
    "leat_argmax_workspace": [_i],
    "leat_argmax": [_p, _i, _i, _p, _i64, _p, _p],
    "leat_probe_read": [_p, _i64, _p, _i, _p],
    "leat_probe_mfma_i8": [_i, _i, _p, _p],
    "leat_glu_matvec_f32": [_i, _p, _p, _i, _i, _p, _i, _p, _f, _i, _p, _p, _p, _p, _p],
}


class LeatError(RuntimeError):
    """A kernel entry point refused its arguments or failed to launch."""


@functools.cache
def lib() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise LeatError(
            f"{LIB_PATH} is not built: run `python -m leat_amd.build` (hipcc, gfx950) first"
        )
    handle = ctypes.CDLL(str(LIB_PATH))
    for name, args in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes, fn.restype = args, ctypes.c_int
    handle.leat_last_error.restype = ctypes.c_char_p
    handle.leat_target.restype = ctypes.c_char_p
    handle.leat_abi_version.restype = ctypes.c_int
    for name in ("leat_matmul_workspace", "leat_attention_workspace", "leat_argmax_workspace"):
        getattr(handle, name).restype = ctypes.c_int64
    return handle


def call(name: str, *args) -> None:
    status = getattr(lib(), name)(*args)
    if status != 0:
        raise LeatError(f"{name}: {lib().leat_last_error().decode()}")


def workspace_bytes(ggml_type: int, rows: int, cols: int, tokens: int, gated: bool) -> int:
    """The workspace a prefill product of this shape splits into on the current device (0: none)."""
    return int(lib().leat_matmul_workspace(int(ggml_type), rows, cols, tokens, int(gated)))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


@functools.cache
def device_ok(index: int) -> bool:
    # the kernels are built for gfx950 alone
    name = torch.cuda.get_device_properties(index).gcnArchName
    return name.split(":")[0] == lib().leat_target().decode()


def require_device(t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise LeatError("the leat_amd kernels take tensors on the GPU (a gfx950 device)")
    if not device_ok(t.device.index if t.device.index is not None else torch.cuda.current_device()):
        raise LeatError("the leat_amd kernels are built for gfx950 (MI355X) only")
