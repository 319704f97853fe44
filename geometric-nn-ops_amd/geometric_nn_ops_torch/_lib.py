"""ctypes binding of libgnn_hip.so (C ABI declared in include/gnn_triangle.h).

The library is loaded lazily on first use. There is no silent fallback: if a CUDA/HIP
tensor reaches a kernel entry point and the library is missing or fails to load, the
call raises RuntimeError naming the path that was tried.
"""

import ctypes
import os
import pathlib
import threading

import torch

LIB_PATH = pathlib.Path(__file__).resolve().parent / "_lib" / "libgnn_hip.so"

GNN_F32, GNN_BF16, GNN_F16 = 0, 1, 2
GNN_PREC_IEEE, GNN_PREC_BF16X3 = 0, 1
GNN_OK, GNN_ERR_ARG, GNN_ERR_UNSUPPORTED, GNN_ERR_WORKSPACE = 0, -1, -2, -3

DTYPE_CODE = {torch.float32: GNN_F32, torch.bfloat16: GNN_BF16, torch.float16: GNN_F16}
PRECISION_CODE = {"ieee": GNN_PREC_IEEE, "bf16x3": GNN_PREC_BF16X3}

I64x3 = ctypes.c_int64 * 3
I64x4 = ctypes.c_int64 * 4


class TriAttnArgs(ctypes.Structure):
    """Mirror of ``gnn_triattn_args``."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("mask", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("row_max", ctypes.c_void_p),
        ("B", ctypes.c_int64),
        ("S", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("D", ctypes.c_int64),
        ("q_stride", I64x4),
        ("k_stride", I64x4),
        ("v_stride", I64x4),
        ("o_stride", I64x4),
        ("bias_stride", I64x4),
        ("mask_stride", I64x3),
        ("scale", ctypes.c_float),
        ("mask_value", ctypes.c_float),
        ("dtype", ctypes.c_int32),
        ("precision", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class TriAttnBwdArgs(ctypes.Structure):
    """Mirror of ``gnn_triattn_bwd_args``."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("dout", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("mask", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("dq", ctypes.c_void_p),
        ("dk", ctypes.c_void_p),
        ("dv", ctypes.c_void_p),
        ("dbias", ctypes.c_void_p),
        ("delta", ctypes.c_void_p),
        ("dbias_ws", ctypes.c_void_p),
        ("dbias_splits", ctypes.c_int32),
        ("B", ctypes.c_int64),
        ("S", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("D", ctypes.c_int64),
        ("q_stride", I64x4),
        ("k_stride", I64x4),
        ("v_stride", I64x4),
        ("o_stride", I64x4),
        ("do_stride", I64x4),
        ("dq_stride", I64x4),
        ("dk_stride", I64x4),
        ("dv_stride", I64x4),
        ("bias_stride", I64x4),
        ("mask_stride", I64x3),
        ("scale", ctypes.c_float),
        ("mask_value", ctypes.c_float),
        ("dtype", ctypes.c_int32),
        ("precision", ctypes.c_int32),
    ]


class TrimulArgs(ctypes.Structure):
    """Mirror of ``gnn_trimul_args``."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("mask", ctypes.c_void_p),
        ("mask_stride", I64x3),
        ("ln_in_w", ctypes.c_void_p),
        ("ln_in_b", ctypes.c_void_p),
        ("p_in_w", ctypes.c_void_p),
        ("p_in_b", ctypes.c_void_p),
        ("g_in_w", ctypes.c_void_p),
        ("g_in_b", ctypes.c_void_p),
        ("ln_out_w", ctypes.c_void_p),
        ("ln_out_b", ctypes.c_void_p),
        ("p_out_w", ctypes.c_void_p),
        ("p_out_b", ctypes.c_void_p),
        ("g_out_w", ctypes.c_void_p),
        ("g_out_b", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("B", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("C", ctypes.c_int64),
        ("Ch", ctypes.c_int64),
        ("eps", ctypes.c_float),
        ("outgoing", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("precision", ctypes.c_int32),
        ("gate", ctypes.c_void_p),
        ("ln_in_channels", ctypes.c_int64),
        ("ln_out_channels", ctypes.c_int64),
    ]


class ApbGateOutArgs(ctypes.Structure):
    """Mirror of ``gnn_apb_gate_out_args``."""

    _fields_ = [
        ("s", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("g_w", ctypes.c_void_p),
        ("g_b", ctypes.c_void_p),
        ("o_w", ctypes.c_void_p),
        ("o_b", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("M", ctypes.c_int64),
        ("Cs", ctypes.c_int64),
        ("D", ctypes.c_int64),
        ("Co", ctypes.c_int64),
        ("s_ld", ctypes.c_int64),
        ("o_ld", ctypes.c_int64),
        ("out_ld", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("precision", ctypes.c_int32),
    ]


class PairBiasArgs(ctypes.Structure):
    """Mirror of ``gnn_pair_bias_args``."""

    _fields_ = [
        ("z", ctypes.c_void_p),
        ("ln_w", ctypes.c_void_p),
        ("proj_w", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("B", ctypes.c_int64),
        ("U", ctypes.c_int64),
        ("V", ctypes.c_int64),
        ("Zc", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("out_stride", I64x3),
        ("eps", ctypes.c_float),
        ("dtype", ctypes.c_int32),
    ]


class LayerNormArgs(ctypes.Structure):
    """Mirror of ``gnn_layernorm_args``."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("dy", ctypes.c_void_p),
        ("weight", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("partial", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("K", ctypes.c_int64),
        ("x_stride", ctypes.c_int64),
        ("dy_stride", ctypes.c_int64),
        ("out_stride", ctypes.c_int64),
        ("eps", ctypes.c_float),
        ("dtype", ctypes.c_int32),
    ]


class GateBwdArgs(ctypes.Structure):
    """Mirror of ``gnn_gate_bwd_args``."""

    _fields_ = [
        ("grad", ctypes.c_void_p),
        ("value", ctypes.c_void_p),
        ("gate_pre", ctypes.c_void_p),
        ("mask", ctypes.c_void_p),
        ("d_value", ctypes.c_void_p),
        ("d_gate_pre", ctypes.c_void_p),
        ("partial", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("K", ctypes.c_int64),
        ("grad_stride", ctypes.c_int64),
        ("value_stride", ctypes.c_int64),
        ("gate_stride", ctypes.c_int64),
        ("mask_stride", ctypes.c_int64),
        ("dv_stride", ctypes.c_int64),
        ("dg_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("gate_is_sigmoid", ctypes.c_int32),
    ]


class TrimulOutBwdArgs(ctypes.Structure):
    """Mirror of ``gnn_trimul_out_bwd_args``."""

    _fields_ = [
        ("o", ctypes.c_void_p),
        ("ln_w", ctypes.c_void_p),
        ("ln_b", ctypes.c_void_p),
        ("p_out_w", ctypes.c_void_p),
        ("p_out_b", ctypes.c_void_p),
        ("gate", ctypes.c_void_p),
        ("dout", ctypes.c_void_p),
        ("on", ctypes.c_void_p),
        ("dy", ctypes.c_void_p),
        ("d_go", ctypes.c_void_p),
        ("d_o", ctypes.c_void_p),
        ("partial", ctypes.c_void_p),
        ("B", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("C", ctypes.c_int64),
        ("Ch", ctypes.c_int64),
        ("dgo_ld", ctypes.c_int64),
        ("eps", ctypes.c_float),
        ("dtype", ctypes.c_int32),
    ]


class TrimulProjBwdArgs(ctypes.Structure):
    """Mirror of ``gnn_trimul_proj_bwd_args``."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("ln_w", ctypes.c_void_p),
        ("ln_b", ctypes.c_void_p),
        ("p_in_w", ctypes.c_void_p),
        ("p_in_b", ctypes.c_void_p),
        ("g_in_w", ctypes.c_void_p),
        ("g_in_b", ctypes.c_void_p),
        ("mask", ctypes.c_void_p),
        ("d_ab", ctypes.c_void_p),
        ("d_p", ctypes.c_void_p),
        ("d_g", ctypes.c_void_p),
        ("z", ctypes.c_void_p),
        ("partial", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("C", ctypes.c_int64),
        ("Ch", ctypes.c_int64),
        ("x_ld", ctypes.c_int64),
        ("dab_ld", ctypes.c_int64),
        ("dl_ld", ctypes.c_int64),
        ("mask_stride", ctypes.c_int64),
        ("eps", ctypes.c_float),
        ("dtype", ctypes.c_int32),
    ]


# Every symbol include/gnn_triangle.h declares, with its ctypes signature.
class TrimulContractBwdArgs(ctypes.Structure):
    """Mirror of ``gnn_trimul_contract_bwd_args``."""

    _fields_ = [
        ("a", ctypes.c_void_p),
        ("b", ctypes.c_void_p),
        ("do_i", ctypes.c_void_p),
        ("do_j", ctypes.c_void_p),
        ("da", ctypes.c_void_p),
        ("db", ctypes.c_void_p),
        ("planes", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class TrimulRelayoutArgs(ctypes.Structure):
    """Mirror of ``gnn_trimul_relayout_args``."""

    _fields_ = [
        ("src", ctypes.c_void_p),
        ("dst", ctypes.c_void_p),
        ("B", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("Ch", ctypes.c_int64),
        ("src_ld", ctypes.c_int64),
        ("dst_ld", ctypes.c_int64),
        ("src_c0", ctypes.c_int64),
        ("dst_c0", ctypes.c_int64),
        ("mode", ctypes.c_int32),
        ("transposed", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


RELAYOUT_PLANES_TO_PIXELS, RELAYOUT_PIXELS_TO_BLOCKED = 0, 1

_SIGNATURES = {
    "gnn_triattn_fwd": (ctypes.c_int, [ctypes.POINTER(TriAttnArgs), ctypes.c_void_p]),
    "gnn_triattn_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(TriAttnArgs)]),
    "gnn_triattn_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(TriAttnArgs), ctypes.c_void_p]),
    "gnn_triattn_bwd": (ctypes.c_int, [ctypes.POINTER(TriAttnBwdArgs), ctypes.c_void_p]),
    "gnn_trimul_workspace_bytes": (
        ctypes.c_size_t,
        [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
         ctypes.POINTER(ctypes.c_size_t)],
    ),
    "gnn_trimul_fwd": (ctypes.c_int, [ctypes.POINTER(TrimulArgs), ctypes.c_void_p]),
    "gnn_trimul_proj": (ctypes.c_int, [ctypes.POINTER(TrimulArgs), ctypes.c_void_p]),
    "gnn_trimul_contract": (ctypes.c_int, [ctypes.POINTER(TrimulArgs), ctypes.c_void_p]),
    "gnn_trimul_out": (ctypes.c_int, [ctypes.POINTER(TrimulArgs), ctypes.c_void_p]),
    "gnn_pair_bias_proj": (ctypes.c_int, [ctypes.POINTER(PairBiasArgs), ctypes.c_void_p]),
    "gnn_apb_gate_out": (ctypes.c_int, [ctypes.POINTER(ApbGateOutArgs), ctypes.c_void_p]),
    "gnn_layernorm_partials": (ctypes.c_int64, [ctypes.c_int64, ctypes.c_int64]),
    "gnn_layernorm_rows": (ctypes.c_int, [ctypes.POINTER(LayerNormArgs), ctypes.c_void_p]),
    "gnn_gate_bwd_partials": (ctypes.c_int64, [ctypes.c_int64, ctypes.c_int64]),
    "gnn_trimul_gate_bwd": (ctypes.c_int, [ctypes.POINTER(GateBwdArgs), ctypes.c_void_p]),
    "gnn_trimul_proj_bwd_partials": (ctypes.c_int64, [ctypes.c_int64]),
    "gnn_trimul_out_bwd_partials": (ctypes.c_int64, [ctypes.c_int64, ctypes.c_int64]),
    "gnn_trimul_out_bwd": (ctypes.c_int, [ctypes.POINTER(TrimulOutBwdArgs), ctypes.c_void_p]),
    "gnn_trimul_proj_bwd": (ctypes.c_int, [ctypes.POINTER(TrimulProjBwdArgs), ctypes.c_void_p]),
    "gnn_trimul_contract_bwd": (ctypes.c_int, [ctypes.POINTER(TrimulContractBwdArgs), ctypes.c_void_p]),
    "gnn_trimul_relayout": (ctypes.c_int, [ctypes.POINTER(TrimulRelayoutArgs), ctypes.c_void_p]),
    "gnn_last_error": (ctypes.c_char_p, []),
    "gnn_version": (ctypes.c_char_p, []),
}
EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib = None


def library_path() -> pathlib.Path:
    override = os.environ.get("GNN_HIP_LIB")
    return pathlib.Path(override) if override else LIB_PATH


def load() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError if it is missing or unloadable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = library_path()
            if not path.exists():
                raise RuntimeError(
                    f"libgnn_hip.so not found at {path}; build it with "
                    "`python geometric-nn-ops_amd/build.py` (no fallback is taken for GPU tensors)"
                )
            try:
                lib = ctypes.CDLL(str(path))
            except OSError as exc:
                raise RuntimeError(f"failed to load {path}: {exc}") from exc
            for name, (res, argtypes) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = argtypes
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    """Raise for a non-zero status from the library, with its message."""
    if rc == GNN_OK:
        return
    msg = load().gnn_last_error().decode(errors="replace")
    if rc == GNN_ERR_ARG:
        raise ValueError(f"{what}: {msg}")
    if rc == GNN_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed with status {rc}: {msg}")


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def call(fn_name: str, args, device: torch.device) -> None:
    """``fn_name(&args, stream)`` on ``device``'s current stream, with ``device`` current for
    the call (the current device is switched only when it differs: the guard costs host time
    on every launch), raising on a non-zero status."""
    fn = getattr(load(), fn_name)
    idx = device.index
    if idx is None or idx == torch.cuda.current_device():
        rc = fn(ctypes.byref(args), ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream))
    else:
        with torch.cuda.device(idx):
            rc = fn(ctypes.byref(args), ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream))
    check(rc, fn_name)


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()
