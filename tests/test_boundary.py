"""The C-ABI boundary on a CPU-only host: libgnn_hip.so loads, exports every function the
header declares, its ctypes struct mirrors have the C layout, and argument errors come
back as status codes + messages before any GPU work is attempted."""

import ctypes
import pathlib
import re
import subprocess

import pytest

from geometric_nn_ops_torch import _lib

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "gnn_triangle.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gnn_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert names, "no declarations parsed from the header"
    for name in names:
        assert hasattr(lib, name), f"{name} declared in gnn_triangle.h but not exported"
    assert set(names) == set(_lib.EXPORTED_SYMBOLS)
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.library_path())],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (gnn_[a-z_0-9]+)", out))
    assert set(names) <= exported


def test_version():
    assert _lib.load().gnn_version().decode().endswith("gfx950")


def _c_layout():
    """offsetof/sizeof of the C structs, from a tiny host program compiled with gcc."""
    src = r"""
    #include <stdio.h>
    #include <stddef.h>
    #include "gnn_triangle.h"
    #define P(T, f) printf(#T "." #f " %zu\n", offsetof(T, f));
    int main(void) {
      printf("gnn_triattn_args %zu\n", sizeof(gnn_triattn_args));
      printf("gnn_trimul_args %zu\n", sizeof(gnn_trimul_args));
      printf("gnn_pair_bias_args %zu\n", sizeof(gnn_pair_bias_args));
      printf("gnn_triattn_bwd_args %zu\n", sizeof(gnn_triattn_bwd_args));
      printf("gnn_layernorm_args %zu\n", sizeof(gnn_layernorm_args));
      printf("gnn_gate_bwd_args %zu\n", sizeof(gnn_gate_bwd_args));
      printf("gnn_trimul_contract_bwd_args %zu\n", sizeof(gnn_trimul_contract_bwd_args));
      printf("gnn_apb_gate_out_args %zu\n", sizeof(gnn_apb_gate_out_args));
      printf("gnn_trimul_proj_bwd_args %zu\n", sizeof(gnn_trimul_proj_bwd_args));
      printf("gnn_trimul_out_bwd_args %zu\n", sizeof(gnn_trimul_out_bwd_args));
      P(gnn_trimul_out_bwd_args, gate) P(gnn_trimul_out_bwd_args, partial) P(gnn_trimul_out_bwd_args, B)
      P(gnn_trimul_out_bwd_args, dgo_ld) P(gnn_trimul_out_bwd_args, eps) P(gnn_trimul_out_bwd_args, dtype)
      P(gnn_trimul_proj_bwd_args, mask) P(gnn_trimul_proj_bwd_args, partial) P(gnn_trimul_proj_bwd_args, rows)
      P(gnn_trimul_proj_bwd_args, mask_stride) P(gnn_trimul_proj_bwd_args, eps) P(gnn_trimul_proj_bwd_args, dtype)
      P(gnn_apb_gate_out_args, o_b) P(gnn_apb_gate_out_args, out) P(gnn_apb_gate_out_args, M)
      P(gnn_apb_gate_out_args, Co) P(gnn_apb_gate_out_args, out_ld) P(gnn_apb_gate_out_args, dtype)
      P(gnn_apb_gate_out_args, precision)
      P(gnn_trimul_contract_bwd_args, do_j) P(gnn_trimul_contract_bwd_args, db)
      P(gnn_trimul_contract_bwd_args, planes) P(gnn_trimul_contract_bwd_args, N) P(gnn_trimul_contract_bwd_args, dtype)
      P(gnn_layernorm_args, partial) P(gnn_layernorm_args, rows) P(gnn_layernorm_args, out_stride)
      P(gnn_layernorm_args, eps) P(gnn_layernorm_args, dtype)
      P(gnn_gate_bwd_args, d_gate_pre) P(gnn_gate_bwd_args, partial) P(gnn_gate_bwd_args, rows) P(gnn_gate_bwd_args, mask_stride)
      P(gnn_gate_bwd_args, dg_stride) P(gnn_gate_bwd_args, dtype) P(gnn_gate_bwd_args, gate_is_sigmoid)
      P(gnn_triattn_args, lse) P(gnn_triattn_args, row_max) P(gnn_triattn_args, D) P(gnn_triattn_args, bias_stride)
      P(gnn_triattn_args, mask_stride) P(gnn_triattn_args, scale) P(gnn_triattn_args, precision)
      P(gnn_trimul_args, mask_stride) P(gnn_trimul_args, workspace_bytes) P(gnn_trimul_args, Ch)
      P(gnn_trimul_args, eps) P(gnn_trimul_args, precision) P(gnn_trimul_args, gate)
      P(gnn_pair_bias_args, out) P(gnn_pair_bias_args, H) P(gnn_pair_bias_args, out_stride)
      P(gnn_pair_bias_args, eps) P(gnn_pair_bias_args, dtype)
      P(gnn_triattn_bwd_args, delta) P(gnn_triattn_bwd_args, dbias_splits) P(gnn_triattn_bwd_args, D) P(gnn_triattn_bwd_args, dv_stride)
      P(gnn_triattn_bwd_args, mask_stride) P(gnn_triattn_bwd_args, scale) P(gnn_triattn_bwd_args, precision)
      return 0;
    }
    """
    return src


def test_ctypes_structs_match_c_layout(tmp_path):
    c = tmp_path / "layout.c"
    c.write_text(_c_layout())
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{ROOT / 'include'}", str(c), "-o", str(exe)], check=True)
    lines = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                                check=True).stdout.splitlines())
    assert int(lines["gnn_triattn_args"]) == ctypes.sizeof(_lib.TriAttnArgs)
    assert int(lines["gnn_trimul_args"]) == ctypes.sizeof(_lib.TrimulArgs)
    assert int(lines["gnn_pair_bias_args"]) == ctypes.sizeof(_lib.PairBiasArgs)
    assert int(lines["gnn_triattn_bwd_args"]) == ctypes.sizeof(_lib.TriAttnBwdArgs)
    assert int(lines["gnn_layernorm_args"]) == ctypes.sizeof(_lib.LayerNormArgs)
    assert int(lines["gnn_gate_bwd_args"]) == ctypes.sizeof(_lib.GateBwdArgs)
    assert int(lines["gnn_trimul_contract_bwd_args"]) == ctypes.sizeof(_lib.TrimulContractBwdArgs)
    assert int(lines["gnn_apb_gate_out_args"]) == ctypes.sizeof(_lib.ApbGateOutArgs)
    assert int(lines["gnn_trimul_proj_bwd_args"]) == ctypes.sizeof(_lib.TrimulProjBwdArgs)
    assert int(lines["gnn_trimul_out_bwd_args"]) == ctypes.sizeof(_lib.TrimulOutBwdArgs)
    classes = {"gnn_triattn_args": _lib.TriAttnArgs, "gnn_trimul_args": _lib.TrimulArgs,
               "gnn_pair_bias_args": _lib.PairBiasArgs, "gnn_triattn_bwd_args": _lib.TriAttnBwdArgs,
               "gnn_layernorm_args": _lib.LayerNormArgs, "gnn_gate_bwd_args": _lib.GateBwdArgs,
               "gnn_trimul_contract_bwd_args": _lib.TrimulContractBwdArgs,
               "gnn_apb_gate_out_args": _lib.ApbGateOutArgs, "gnn_trimul_proj_bwd_args": _lib.TrimulProjBwdArgs,
               "gnn_trimul_out_bwd_args": _lib.TrimulOutBwdArgs}
    for key, val in lines.items():
        if "." not in key:
            continue
        struct, field = key.split(".")
        cls = classes[struct]
        assert getattr(cls, field).offset == int(val), key


def test_null_args_are_rejected_without_a_gpu():
    lib = _lib.load()
    assert lib.gnn_triattn_fwd(None, None) == _lib.GNN_ERR_ARG
    assert b"NULL" in lib.gnn_last_error()
    assert lib.gnn_trimul_fwd(None, None) == _lib.GNN_ERR_ARG


def test_triattn_argument_errors():
    lib = _lib.load()
    a = _lib.TriAttnArgs()
    assert lib.gnn_triattn_fwd(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"required" in lib.gnn_last_error()
    a.q = a.k = a.v = a.o = 4096
    a.B = a.S = a.N = a.H = 1
    a.D = 12
    assert lib.gnn_triattn_fwd(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"multiple of 8" in lib.gnn_last_error()
    a.D = 16
    a.q_stride = _lib.I64x4(16, 16, 12, 16)
    assert lib.gnn_triattn_fwd(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"strides" in lib.gnn_last_error()
    with pytest.raises(ValueError, match="strides"):
        _lib.check(_lib.GNN_ERR_ARG, "gnn_triattn_fwd")


def test_triattn_head_dim_limits():
    """Head dims up to 256 for 16-bit inputs and 128 for fp32; wider ones are refused
    before any launch."""
    lib = _lib.load()
    a = _lib.TriAttnArgs()
    a.q = a.k = a.v = a.o = 4096
    a.B, a.S, a.N, a.H = 1, 2, 40, 2
    for D, dtype, msg in ((264, _lib.GNN_BF16, b"head dim > 256"), (136, _lib.GNN_F32, b"fp32 head dim > 128")):
        a.D, a.dtype = D, dtype
        for st in ("q_stride", "k_stride", "v_stride", "o_stride"):
            setattr(a, st, _lib.I64x4(2 * 40 * 2 * D, 40 * 2 * D, 2 * D, D))
        assert lib.gnn_triattn_fwd(ctypes.byref(a), None) == _lib.GNN_ERR_UNSUPPORTED
        assert msg in lib.gnn_last_error()


def test_triattn_workspace():
    """The 16-bit row path with a pair bias needs caller scratch for the bias in fragment
    order (4 KB per 32-query x 64-key tile per (batch, head)); other calls need none, and a
    missing or short workspace is refused before any launch."""
    lib = _lib.load()
    a = _lib.TriAttnArgs()
    a.q = a.k = a.v = a.o = 4096
    a.B, a.S, a.N, a.H, a.D = 2, 3, 100, 4, 32
    for st in ("q_stride", "k_stride", "v_stride", "o_stride"):
        setattr(a, st, _lib.I64x4(3 * 100 * 128, 100 * 128, 128, 32))
    a.dtype = _lib.GNN_BF16
    assert lib.gnn_triattn_workspace_bytes(ctypes.byref(a)) == 0  # no bias
    a.bias = 8192
    a.bias_stride = _lib.I64x4(4 * 100 * 100, 100 * 100, 1, 100)  # a transposed view is fine here
    need = 2 * 4 * 4 * 2 * 4096  # B * H * ceil(100/32) * ceil(100/64) tiles of 4 KB
    assert lib.gnn_triattn_workspace_bytes(ctypes.byref(a)) == need
    assert lib.gnn_triattn_fwd(ctypes.byref(a), None) == _lib.GNN_ERR_WORKSPACE
    a.workspace, a.workspace_bytes = 1 << 20, need - 1
    assert lib.gnn_triattn_fwd(ctypes.byref(a), None) == _lib.GNN_ERR_WORKSPACE
    assert b"workspace" in lib.gnn_last_error()
    a.dtype = _lib.GNN_F32  # the tiled kernel reads the bias in place
    assert lib.gnn_triattn_workspace_bytes(ctypes.byref(a)) == 0
    assert lib.gnn_triattn_fwd(ctypes.byref(a), None) == _lib.GNN_ERR_ARG  # ... with unit key stride
    assert b"unit key stride" in lib.gnn_last_error()


def test_triattn_noalloc_rejects_calls_beyond_its_static_scratch():
    """The allocation-free entry point refuses, before touching the device, a call whose bias
    tiles exceed its 16 MiB array (here B * H * ceil(N/32) * ceil(N/64) * 4 KB = 32 MiB)."""
    lib = _lib.load()
    a = _lib.TriAttnArgs()
    a.q = a.k = a.v = a.o = 4096
    a.B, a.S, a.N, a.H, a.D = 1, 1, 1024, 16, 32
    for st in ("q_stride", "k_stride", "v_stride", "o_stride"):
        setattr(a, st, _lib.I64x4(1024 * 1024 * 16 * 32, 1024 * 16 * 32, 16 * 32, 32))
    a.bias = 8192
    a.bias_stride = _lib.I64x4(16 * 1024 * 1024, 1024 * 1024, 1024, 1)
    a.dtype = _lib.GNN_BF16
    assert lib.gnn_triattn_workspace_bytes(ctypes.byref(a)) == 32 << 20
    assert lib.gnn_triattn_fwd_noalloc(ctypes.byref(a), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"16 MiB" in lib.gnn_last_error()


def test_trimul_argument_errors_and_workspace():
    lib = _lib.load()
    off = (ctypes.c_size_t * 4)()
    n = lib.gnn_trimul_workspace_bytes(1, 512, 128, 128, _lib.GNN_BF16, off)
    plane = 128 * 512 * 512 * 2
    # a, b, o, then the gate region last (a caller with its own gate buffer stops at off[2])
    assert off[0] == 0 and off[1] == plane and off[3] == 2 * plane
    assert off[2] == 3 * plane and n == off[2] + 512 * 512 * 128 * 2
    assert lib.gnn_trimul_workspace_bytes(1, 100, 32, 32, _lib.GNN_F32, None) % 256 == 0
    a = _lib.TrimulArgs()
    assert lib.gnn_trimul_fwd(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    a.x = a.out = a.p_in_w = a.g_in_w = a.p_out_w = a.g_out_w = 4096
    a.B, a.N, a.C, a.Ch = 1, 8, 48, 32
    a.dtype = _lib.GNN_BF16
    assert lib.gnn_trimul_proj(ctypes.byref(a), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"multiples of 32" in lib.gnn_last_error()
    a.C = 32
    a.workspace = 4096
    a.workspace_bytes = 10
    assert lib.gnn_trimul_contract(ctypes.byref(a), None) == _lib.GNN_ERR_WORKSPACE
    # with its own gate buffer the workspace may stop at the gate offset, not before it
    off = (ctypes.c_size_t * 4)()
    lib.gnn_trimul_workspace_bytes(1, 8, 32, 32, _lib.GNN_BF16, off)
    a.gate = 8192
    a.workspace_bytes = off[2] - 1
    assert lib.gnn_trimul_contract(ctypes.byref(a), None) == _lib.GNN_ERR_WORKSPACE
    a.gate = 8200
    assert lib.gnn_trimul_contract(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"16-byte aligned" in lib.gnn_last_error()
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.check(_lib.GNN_ERR_WORKSPACE, "gnn_trimul_contract")


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setenv("GNN_HIP_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(RuntimeError, match="not found"):
        _lib.load()
    monkeypatch.delenv("GNN_HIP_LIB")
    monkeypatch.setattr(_lib, "_lib", None)
    _lib.load()


def test_pair_bias_argument_errors():
    lib = _lib.load()
    assert lib.gnn_pair_bias_proj(None, None) == _lib.GNN_ERR_ARG
    a = _lib.PairBiasArgs()
    assert lib.gnn_pair_bias_proj(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"required" in lib.gnn_last_error()
    a.z = a.proj_w = a.out = 4096
    a.B, a.U, a.V, a.H = 1, 8, 8, 4
    a.Zc = 0
    assert lib.gnn_pair_bias_proj(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"positive" in lib.gnn_last_error()
    a.Zc = 12
    assert lib.gnn_pair_bias_proj(ctypes.byref(a), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"multiple of 8" in lib.gnn_last_error()
    a.Zc, a.H = 256, 64
    assert lib.gnn_pair_bias_proj(ctypes.byref(a), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"8192" in lib.gnn_last_error()
    a.z = 4100
    assert lib.gnn_pair_bias_proj(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"aligned" in lib.gnn_last_error()


def test_triattn_bwd_argument_errors():
    lib = _lib.load()
    assert lib.gnn_triattn_bwd(None, None) == _lib.GNN_ERR_ARG
    a = _lib.TriAttnBwdArgs()
    assert lib.gnn_triattn_bwd(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"required" in lib.gnn_last_error()
    a.q = a.k = a.v = a.o = a.dout = a.lse = a.dq = a.dk = a.dv = a.delta = 4096
    a.B = a.S = a.N = a.H = 1
    a.D = 12
    assert lib.gnn_triattn_bwd(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"multiple of 8" in lib.gnn_last_error()
    a.D = 136  # above the 128 the chunked kernels cover (refused before the dtype is looked at)
    assert lib.gnn_triattn_bwd(ctypes.byref(a), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"head dim" in lib.gnn_last_error()
    a.D = 96  # fp32 tiles take twice the LDS: fp32 head dims up to 64
    a.dtype = _lib.GNN_F32
    assert lib.gnn_triattn_bwd(ctypes.byref(a), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"fp32 head dim" in lib.gnn_last_error()
    a.D = 32
    a.dtype = 7  # no such dtype code
    assert lib.gnn_triattn_bwd(ctypes.byref(a), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"bf16 / fp16 / fp32" in lib.gnn_last_error()


def test_trimul_backward_helper_argument_errors():
    lib = _lib.load()
    assert lib.gnn_layernorm_rows(None, None) == _lib.GNN_ERR_ARG
    a = _lib.LayerNormArgs()
    assert lib.gnn_layernorm_rows(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"required" in lib.gnn_last_error()
    a.x = a.out = 4096
    a.rows, a.K, a.x_stride, a.out_stride = 4, 96, 96, 64
    assert lib.gnn_layernorm_rows(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"stride" in lib.gnn_last_error()
    a.out_stride = 96
    a.dy, a.dy_stride, a.bias = 4096, 96, 4096
    assert lib.gnn_layernorm_rows(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"forward-only" in lib.gnn_last_error()
    a.bias = None
    a.K = a.x_stride = a.out_stride = a.dy_stride = 48
    assert lib.gnn_layernorm_rows(ctypes.byref(a), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"multiple of 32" in lib.gnn_last_error()
    # rows wider than 512: forward only, at most 8192, 16-byte aligned rows
    a.K = a.x_stride = a.out_stride = a.dy_stride = 1024
    assert lib.gnn_layernorm_rows(ctypes.byref(a), None) == _lib.GNN_ERR_UNSUPPORTED  # a backward
    assert b"8192 for the forward" in lib.gnn_last_error()
    a.dy = None
    a.K = a.x_stride = a.out_stride = 8224
    assert lib.gnn_layernorm_rows(ctypes.byref(a), None) == _lib.GNN_ERR_UNSUPPORTED
    a.K, a.x_stride, a.out_stride, a.x = 1024, 1024, 1024, 4098
    assert lib.gnn_layernorm_rows(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"16-byte aligned" in lib.gnn_last_error()
    assert lib.gnn_layernorm_partials(1 << 20, 128) == 4096
    assert lib.gnn_layernorm_partials(40, 128) == 2
    assert lib.gnn_gate_bwd_partials(1 << 20, 256) == 1024
    assert lib.gnn_gate_bwd_partials(100, 128) == 7
    assert lib.gnn_gate_bwd_partials(100, 96) == 0  # 12 chunks per row do not divide 256

    assert lib.gnn_trimul_gate_bwd(None, None) == _lib.GNN_ERR_ARG
    g = _lib.GateBwdArgs()
    assert lib.gnn_trimul_gate_bwd(ctypes.byref(g), None) == _lib.GNN_ERR_ARG
    assert b"required" in lib.gnn_last_error()
    g.grad = g.value = g.gate_pre = g.d_value = g.d_gate_pre = 4096
    g.rows, g.K = 4, 64
    g.grad_stride = g.value_stride = g.gate_stride = g.dv_stride = g.dg_stride = 64
    g.grad_stride = 60
    assert lib.gnn_trimul_gate_bwd(ctypes.byref(g), None) == _lib.GNN_ERR_ARG
    g.grad_stride, g.value = 64, 4098
    assert lib.gnn_trimul_gate_bwd(ctypes.byref(g), None) == _lib.GNN_ERR_ARG
    assert b"aligned" in lib.gnn_last_error()
    g.value = 4096
    g.K = 12
    g.grad_stride = g.value_stride = g.gate_stride = g.dv_stride = g.dg_stride = 16
    assert lib.gnn_trimul_gate_bwd(ctypes.byref(g), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"multiple of 8" in lib.gnn_last_error()

    assert lib.gnn_trimul_proj_bwd(None, None) == _lib.GNN_ERR_ARG
    pb = _lib.TrimulProjBwdArgs()
    assert lib.gnn_trimul_proj_bwd(ctypes.byref(pb), None) == _lib.GNN_ERR_ARG
    assert b"required" in lib.gnn_last_error()
    pb.x = pb.p_in_w = pb.g_in_w = pb.d_ab = pb.d_p = pb.d_g = pb.z = pb.partial = 4096
    pb.rows, pb.C, pb.Ch = 100, 128, 64
    pb.x_ld, pb.dab_ld, pb.dl_ld = 128, 100, 384  # d_ab rows shorter than 2 c_hidden
    assert lib.gnn_trimul_proj_bwd(ctypes.byref(pb), None) == _lib.GNN_ERR_ARG
    assert b"stride" in lib.gnn_last_error()
    pb.dab_ld, pb.d_g = 128, 4100
    assert lib.gnn_trimul_proj_bwd(ctypes.byref(pb), None) == _lib.GNN_ERR_ARG
    assert b"aligned" in lib.gnn_last_error()
    pb.d_g, pb.dtype = 4096, _lib.GNN_F32
    assert lib.gnn_trimul_proj_bwd(ctypes.byref(pb), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"bf16 / fp16" in lib.gnn_last_error()
    pb.dtype, pb.C, pb.x_ld = _lib.GNN_BF16, 96, 96
    assert lib.gnn_trimul_proj_bwd(ctypes.byref(pb), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"C must be 64 or 128" in lib.gnn_last_error()
    assert lib.gnn_trimul_proj_bwd_partials(100) == 2
    assert lib.gnn_trimul_proj_bwd_partials(1 << 20) == 512

    assert lib.gnn_trimul_out_bwd(None, None) == _lib.GNN_ERR_ARG
    ob = _lib.TrimulOutBwdArgs()
    assert lib.gnn_trimul_out_bwd(ctypes.byref(ob), None) == _lib.GNN_ERR_ARG
    assert b"required" in lib.gnn_last_error()
    ob.o = ob.p_out_w = ob.gate = ob.dout = ob.on = ob.dy = ob.d_go = ob.d_o = ob.partial = 4096
    ob.B, ob.N, ob.C, ob.Ch, ob.dgo_ld = 1, 40, 128, 128, 100
    assert lib.gnn_trimul_out_bwd(ctypes.byref(ob), None) == _lib.GNN_ERR_ARG
    assert b"d_go rows" in lib.gnn_last_error()
    ob.dgo_ld, ob.dy = 640, 4104
    assert lib.gnn_trimul_out_bwd(ctypes.byref(ob), None) == _lib.GNN_ERR_ARG
    assert b"aligned" in lib.gnn_last_error()
    ob.dy, ob.Ch = 4096, 96
    assert lib.gnn_trimul_out_bwd(ctypes.byref(ob), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"c_hidden 32, 64 or 128" in lib.gnn_last_error()
    ob.Ch, ob.dtype = 128, _lib.GNN_F32
    assert lib.gnn_trimul_out_bwd(ctypes.byref(ob), None) == _lib.GNN_ERR_UNSUPPORTED
    assert lib.gnn_trimul_out_bwd_partials(1, 40) == 40
    assert lib.gnn_trimul_out_bwd_partials(1, 512) == 512

    assert lib.gnn_trimul_contract_bwd(None, None) == _lib.GNN_ERR_ARG
    cb = _lib.TrimulContractBwdArgs()
    assert lib.gnn_trimul_contract_bwd(ctypes.byref(cb), None) == _lib.GNN_ERR_ARG
    assert b"required" in lib.gnn_last_error()
    cb.a = cb.b = cb.do_i = cb.do_j = cb.da = cb.db = 4096
    cb.planes, cb.N, cb.dtype = 4, 64, _lib.GNN_F32
    assert lib.gnn_trimul_contract_bwd(ctypes.byref(cb), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"16-bit" in lib.gnn_last_error()
    cb.dtype, cb.N = _lib.GNN_BF16, 0
    assert lib.gnn_trimul_contract_bwd(ctypes.byref(cb), None) == _lib.GNN_ERR_ARG
    cb.N, cb.db = 64, 4104
    assert lib.gnn_trimul_contract_bwd(ctypes.byref(cb), None) == _lib.GNN_ERR_ARG
    assert b"aligned" in lib.gnn_last_error()


def test_apb_gate_out_argument_errors():
    """The fused gate / output projection refuses bad arguments before any launch."""
    lib = _lib.load()
    assert lib.gnn_apb_gate_out(None, None) == _lib.GNN_ERR_ARG
    a = _lib.ApbGateOutArgs()
    assert lib.gnn_apb_gate_out(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"required" in lib.gnn_last_error()
    a.s = a.o = a.g_w = a.o_w = a.out = 4096
    a.M, a.Cs, a.D, a.Co = 10, 64, 64, 64
    a.s_ld = a.o_ld = a.out_ld = 64
    a.dtype = _lib.GNN_BF16
    a.Cs = a.s_ld = 48
    assert lib.gnn_apb_gate_out(ctypes.byref(a), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"multiples of 32" in lib.gnn_last_error()
    a.Cs, a.s_ld = 64, 60
    assert lib.gnn_apb_gate_out(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"pitch" in lib.gnn_last_error()
    a.s_ld = 64
    a.s = 4098
    assert lib.gnn_apb_gate_out(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
    assert b"aligned" in lib.gnn_last_error()
    a.s = 4096
    a.Cs = a.D = a.s_ld = a.o_ld = 2048
    assert lib.gnn_apb_gate_out(ctypes.byref(a), None) == _lib.GNN_ERR_UNSUPPORTED
    assert b"LDS" in lib.gnn_last_error()
    a.dtype = 7
    assert lib.gnn_apb_gate_out(ctypes.byref(a), None) == _lib.GNN_ERR_ARG
