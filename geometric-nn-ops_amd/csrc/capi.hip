// extern "C" entry points of libgnn_hip.so (declared in include/gnn_triangle.h): argument
// validation, the thread-local error message, and dispatch to the kernel launchers.
#include <stdio.h>
#include <string.h>

#include <string>

#include "gnn_internal.hpp"

namespace gnn {

static thread_local std::string g_last_error;

int set_error(int code, const char* msg) {
  g_last_error = msg;
  return code;
}

int persistent_grid(const void* fn, int threads, size_t smem) {
  int dev = 0, ncu = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu < 1)
    ncu = 1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, smem) != hipSuccess || per_cu < 1)
    per_cu = 1;
  return ncu * per_cu;
}

static int hip_status(hipError_t e, const char* who) {
  if (e == hipSuccess) return GNN_OK;
  char buf[256];
  snprintf(buf, sizeof buf, "%s: HIP error %d (%s)", who, (int)e, hipGetErrorString(e));
  g_last_error = buf;
  return (int)e;
}

static bool aligned(const void* p, size_t n) { return ((uintptr_t)p % n) == 0; }

// caller_workspace: the caller provides the scratch (gnn_triattn_fwd); false for the entry
// point whose scratch is the library's static array.
static int check_triattn(const gnn_triattn_args& a, bool caller_workspace = true) {
  if (!a.q || !a.k || !a.v || !a.o)
    return set_error(GNN_ERR_ARG, "triangle_attention: q, k, v and o are required");
  if (a.B < 1 || a.S < 1 || a.N < 1 || a.H < 1 || a.D < 1)
    return set_error(GNN_ERR_ARG, "triangle_attention: B, N_seq, N_res, H and D must be positive");
  if (a.dtype != GNN_BF16 && a.dtype != GNN_F16 && a.dtype != GNN_F32)
    return set_error(GNN_ERR_ARG, "triangle_attention: unknown dtype");
  if (a.D % 8 != 0)
    return set_error(GNN_ERR_ARG, "triangle_attention: D must be a multiple of 8 (pad on the host)");
  const int64_t* st[4] = {a.q_stride, a.k_stride, a.v_stride, a.o_stride};
  const void* ptr[4] = {a.q, a.k, a.v, a.o};
  for (int t = 0; t < 4; ++t) {
    if (!aligned(ptr[t], 16))
      return set_error(GNN_ERR_ARG, "triangle_attention: q/k/v/o must be 16-byte aligned");
    for (int d = 0; d < 4; ++d)
      if (st[t][d] % 8 != 0)
        return set_error(GNN_ERR_ARG, "triangle_attention: q/k/v/o strides must be multiples of 8 elements");
  }
  if (a.bias && !triattn_row_applicable(a)) {
    if (a.bias_stride[3] != 1 || a.bias_stride[2] % 8 != 0 || !aligned(a.bias, 16))
      return set_error(GNN_ERR_ARG,
                       "triangle_attention: bias needs unit key stride, a query stride that is a multiple "
                       "of 8 and 16-byte alignment");
  }
  const size_t need = triattn_row_applicable(a) ? triattn_row_workspace_bytes(a) : 0;
  if (caller_workspace && need && (!a.workspace || a.workspace_bytes < need || !aligned(a.workspace, 16)))
    return set_error(GNN_ERR_WORKSPACE,
                     "triangle_attention: workspace missing, smaller than gnn_triattn_workspace_bytes() or "
                     "not 16-byte aligned");
  return GNN_OK;
}

}  // namespace gnn

using namespace gnn;

extern "C" {

int gnn_triattn_fwd(const gnn_triattn_args* args, void* stream) {
  if (!args) return set_error(GNN_ERR_ARG, "triangle_attention: args is NULL");
  if (int rc = check_triattn(*args)) return rc;
  int rc = triattn_fwd(*args, (hipStream_t)stream);
  if (rc < 0) return rc;
  return hip_status((hipError_t)rc, "triangle_attention");
}

int gnn_triattn_fwd_noalloc(const gnn_triattn_args* args, void* stream) {
  if (!args) return set_error(GNN_ERR_ARG, "triangle_attention: args is NULL");
  if (int rc = check_triattn(*args, false)) return rc;
  int rc = triattn_fwd_noalloc(*args, (hipStream_t)stream);
  if (rc < 0) return rc;
  return hip_status((hipError_t)rc, "triangle_attention (no-alloc)");
}

size_t gnn_triattn_workspace_bytes(const gnn_triattn_args* args) {
  if (!args) return 0;
  return triattn_row_applicable(*args) ? triattn_row_workspace_bytes(*args) : 0;
}

int gnn_triattn_bwd(const gnn_triattn_bwd_args* args, void* stream) {
  if (!args) return set_error(GNN_ERR_ARG, "triangle_attention backward: args is NULL");
  const gnn_triattn_bwd_args& a = *args;
  if (!a.q || !a.k || !a.v || !a.o || !a.dout || !a.lse || !a.dq || !a.dk || !a.dv || !a.delta)
    return set_error(GNN_ERR_ARG, "triangle_attention backward: q, k, v, o, dout, lse, dq, dk, dv and delta are required");
  if (a.B < 1 || a.S < 1 || a.N < 1 || a.H < 1 || a.D < 1)
    return set_error(GNN_ERR_ARG, "triangle_attention backward: B, N_seq, N_res, H and D must be positive");
  if (a.D % 8 != 0)
    return set_error(GNN_ERR_ARG, "triangle_attention backward: D must be a multiple of 8 (pad on the host)");
  const int64_t* st[5] = {a.q_stride, a.k_stride, a.v_stride, a.o_stride, a.do_stride};
  const void* ptr[5] = {a.q, a.k, a.v, a.o, a.dout};
  for (int t = 0; t < 5; ++t) {
    if (!aligned(ptr[t], 16))
      return set_error(GNN_ERR_ARG, "triangle_attention backward: q/k/v/o/dout must be 16-byte aligned");
    for (int d = 0; d < 4; ++d)
      if (st[t][d] % 8 != 0)
        return set_error(GNN_ERR_ARG, "triangle_attention backward: q/k/v/o/dout strides must be multiples of 8 elements");
  }
  if (a.bias && (a.bias_stride[3] != 1 || a.bias_stride[2] % 8 != 0 || !aligned(a.bias, 16)))
    return set_error(GNN_ERR_ARG, "triangle_attention backward: bias needs unit key stride, a query stride that is a "
                                  "multiple of 8 and 16-byte alignment");
  int rc = triattn_bwd(a, (hipStream_t)stream);
  if (rc < 0) return rc;
  return hip_status((hipError_t)rc, "triangle_attention backward");
}

size_t gnn_trimul_workspace_bytes(int64_t B, int64_t N, int64_t C, int64_t Ch, int32_t dtype,
                                  size_t off[4]) {
  const TrimulLayout L = trimul_layout(B, N, C, Ch, dtype);
  if (off) {
    off[0] = L.off_a;
    off[1] = L.off_b;
    off[2] = L.off_g;
    off[3] = L.off_o;
  }
  return L.total;
}

static int trimul_stage(const gnn_trimul_args* args, void* stream, int which) {
  if (!args) return set_error(GNN_ERR_ARG, "trimul: args is NULL");
  hipStream_t st = (hipStream_t)stream;
  int rc = GNN_OK;
  if (which & 1) rc = trimul_proj(*args, st);
  if (rc == GNN_OK && (which & 2)) rc = trimul_contract(*args, st);
  if (rc == GNN_OK && (which & 4)) rc = trimul_out(*args, st);
  if (rc < 0) return rc;
  return hip_status((hipError_t)rc, "trimul");
}

int gnn_trimul_fwd(const gnn_trimul_args* args, void* stream) { return trimul_stage(args, stream, 7); }
int gnn_trimul_proj(const gnn_trimul_args* args, void* stream) { return trimul_stage(args, stream, 1); }
int gnn_trimul_contract(const gnn_trimul_args* args, void* stream) {
  return trimul_stage(args, stream, 2);
}
int gnn_trimul_out(const gnn_trimul_args* args, void* stream) { return trimul_stage(args, stream, 4); }

int gnn_pair_bias_proj(const gnn_pair_bias_args* args, void* stream) {
  if (!args) return set_error(GNN_ERR_ARG, "pair_bias_proj: args is NULL");
  const gnn_pair_bias_args& a = *args;
  if (!a.z || !a.proj_w || !a.out)
    return set_error(GNN_ERR_ARG, "pair_bias_proj: z, proj_w and out are required");
  if (a.B < 1 || a.U < 1 || a.V < 1 || a.Zc < 1 || a.H < 1)
    return set_error(GNN_ERR_ARG, "pair_bias_proj: B, U, V, c_z and H must be positive");
  if (!aligned(a.z, 16))
    return set_error(GNN_ERR_ARG, "pair_bias_proj: z must be 16-byte aligned");
  int rc = pair_bias_proj(a, (hipStream_t)stream);
  if (rc < 0) return rc;
  return hip_status((hipError_t)rc, "pair_bias_proj");
}

int gnn_apb_gate_out(const gnn_apb_gate_out_args* args, void* stream) {
  if (!args) return set_error(GNN_ERR_ARG, "apb_gate_out: args is NULL");
  const gnn_apb_gate_out_args& a = *args;
  if (!a.s || !a.o || !a.g_w || !a.o_w || !a.out)
    return set_error(GNN_ERR_ARG, "apb_gate_out: s, o, g_w, o_w and out are required");
  if (a.M < 1 || a.Cs < 1 || a.D < 1 || a.Co < 1)
    return set_error(GNN_ERR_ARG, "apb_gate_out: M, c_s, the attention width and c_out must be positive");
  if (a.dtype != GNN_BF16 && a.dtype != GNN_F16 && a.dtype != GNN_F32)
    return set_error(GNN_ERR_ARG, "apb_gate_out: unknown dtype");
  const int64_t e = a.dtype == GNN_F32 ? 4 : 2;
  const void* ptrs[] = {a.s, a.o, a.g_w, a.o_w, a.out};
  for (const void* p : ptrs)
    if (!aligned(p, 16)) return set_error(GNN_ERR_ARG, "apb_gate_out: tensors must be 16-byte aligned");
  if ((a.s_ld * e) % 16 || (a.o_ld * e) % 16 || (a.out_ld * e) % 16 || a.s_ld < a.Cs || a.o_ld < a.D ||
      a.out_ld < a.Co)
    return set_error(GNN_ERR_ARG, "apb_gate_out: row pitches must cover the rows and be multiples of 16 bytes");
  int rc = apb_gate_out(a, (hipStream_t)stream);
  if (rc < 0) return rc;
  return hip_status((hipError_t)rc, "apb_gate_out");
}

int64_t gnn_layernorm_partials(int64_t rows, int64_t K) { return layernorm_partials(rows, K); }

int gnn_layernorm_rows(const gnn_layernorm_args* args, void* stream) {
  if (!args) return set_error(GNN_ERR_ARG, "layernorm_rows: args is NULL");
  const gnn_layernorm_args& a = *args;
  if (!a.x || !a.out) return set_error(GNN_ERR_ARG, "layernorm_rows: x and out are required");
  if (a.rows < 1 || a.K < 1) return set_error(GNN_ERR_ARG, "layernorm_rows: rows and K must be positive");
  if (a.x_stride < a.K || a.out_stride < a.K || (a.dy && a.dy_stride < a.K))
    return set_error(GNN_ERR_ARG, "layernorm_rows: a row stride is smaller than K");
  if (a.dy && a.bias) return set_error(GNN_ERR_ARG, "layernorm_rows: bias is a forward-only argument");
  int rc = layernorm_rows(a, (hipStream_t)stream);
  if (rc < 0) return rc;
  return hip_status((hipError_t)rc, "layernorm_rows");
}

int64_t gnn_gate_bwd_partials(int64_t rows, int64_t K) { return gate_bwd_partials(rows, K); }

int gnn_trimul_gate_bwd(const gnn_gate_bwd_args* args, void* stream) {
  if (!args) return set_error(GNN_ERR_ARG, "trimul_gate_bwd: args is NULL");
  const gnn_gate_bwd_args& a = *args;
  if (!a.grad || !a.value || !a.gate_pre || !a.d_value || !a.d_gate_pre)
    return set_error(GNN_ERR_ARG, "trimul_gate_bwd: grad, value, gate_pre, d_value and d_gate_pre are required");
  if (a.rows < 1 || a.K < 1) return set_error(GNN_ERR_ARG, "trimul_gate_bwd: rows and K must be positive");
  const int64_t st[5] = {a.grad_stride, a.value_stride, a.gate_stride, a.dv_stride, a.dg_stride};
  const void* ptr[5] = {a.grad, a.value, a.gate_pre, a.d_value, a.d_gate_pre};
  const int64_t esz = a.dtype == GNN_F32 ? 4 : 2;
  for (int i = 0; i < 5; ++i) {
    if (st[i] < a.K) return set_error(GNN_ERR_ARG, "trimul_gate_bwd: a row stride is smaller than K");
    if ((st[i] * esz) % 16 != 0 || !aligned(ptr[i], 16))
      return set_error(GNN_ERR_ARG, "trimul_gate_bwd: rows must be 16-byte aligned");
  }
  int rc = gate_bwd(a, (hipStream_t)stream);
  if (rc < 0) return rc;
  return hip_status((hipError_t)rc, "trimul_gate_bwd");
}

int64_t gnn_trimul_out_bwd_partials(int64_t B, int64_t N) { return trimul_out_bwd_partials(B, N); }

int gnn_trimul_out_bwd(const gnn_trimul_out_bwd_args* args, void* stream) {
  if (!args) return set_error(GNN_ERR_ARG, "trimul_out_bwd: args is NULL");
  const gnn_trimul_out_bwd_args& a = *args;
  if (!a.o || !a.p_out_w || !a.gate || !a.dout || !a.on || !a.dy || !a.d_go || !a.d_o || !a.partial)
    return set_error(GNN_ERR_ARG, "trimul_out_bwd: o, p_out_w, gate, dout, on, dy, d_go, d_o and partial are required");
  if (a.B < 1 || a.N < 1 || a.C < 1 || a.Ch < 1)
    return set_error(GNN_ERR_ARG, "trimul_out_bwd: B, N, C and c_hidden must be positive");
  if (a.dgo_ld < a.C || (a.dgo_ld * 2) % 16 != 0)
    return set_error(GNN_ERR_ARG, "trimul_out_bwd: d_go rows must cover C and be 16-byte aligned");
  const void* ptr[9] = {a.o, a.p_out_w, a.gate, a.dout, a.on, a.dy, a.d_go, a.d_o, a.partial};
  for (const void* q : ptr)
    if (!aligned(q, 16)) return set_error(GNN_ERR_ARG, "trimul_out_bwd: tensors must be 16-byte aligned");
  int rc = trimul_out_bwd(a, (hipStream_t)stream);
  if (rc < 0) return rc;
  return hip_status((hipError_t)rc, "trimul_out_bwd");
}

int64_t gnn_trimul_proj_bwd_partials(int64_t rows) { return trimul_proj_bwd_partials(rows); }

int gnn_trimul_proj_bwd(const gnn_trimul_proj_bwd_args* args, void* stream) {
  if (!args) return set_error(GNN_ERR_ARG, "trimul_proj_bwd: args is NULL");
  const gnn_trimul_proj_bwd_args& a = *args;
  if (!a.x || !a.p_in_w || !a.g_in_w || !a.d_ab || !a.d_p || !a.d_g || !a.z || !a.partial)
    return set_error(GNN_ERR_ARG, "trimul_proj_bwd: x, p_in_w, g_in_w, d_ab, d_p, d_g, z and partial are required");
  if (a.rows < 1 || a.C < 1 || a.Ch < 1)
    return set_error(GNN_ERR_ARG, "trimul_proj_bwd: rows, C and c_hidden must be positive");
  if (a.x_ld < a.C || a.dab_ld < 2 * a.Ch || a.dl_ld < 2 * a.Ch || a.mask_stride < 0)
    return set_error(GNN_ERR_ARG, "trimul_proj_bwd: a row stride is smaller than its row");
  const int64_t st[3] = {a.x_ld, a.dab_ld, a.dl_ld};
  for (int64_t v : st)
    if ((v * 2) % 16 != 0) return set_error(GNN_ERR_ARG, "trimul_proj_bwd: rows must be 16-byte aligned");
  const void* ptr[6] = {a.x, a.d_ab, a.d_p, a.d_g, a.z, a.p_in_w};
  for (const void* q : ptr)
    if (!aligned(q, 16)) return set_error(GNN_ERR_ARG, "trimul_proj_bwd: tensors must be 16-byte aligned");
  if (!aligned(a.g_in_w, 16)) return set_error(GNN_ERR_ARG, "trimul_proj_bwd: tensors must be 16-byte aligned");
  int rc = trimul_proj_bwd(a, (hipStream_t)stream);
  if (rc < 0) return rc;
  return hip_status((hipError_t)rc, "trimul_proj_bwd");
}

int gnn_trimul_contract_bwd(const gnn_trimul_contract_bwd_args* args, void* stream) {
  if (!args) return set_error(GNN_ERR_ARG, "trimul_contract_bwd: args is NULL");
  const gnn_trimul_contract_bwd_args& a = *args;
  if (!a.a || !a.b || !a.do_i || !a.do_j || !a.da || !a.db)
    return set_error(GNN_ERR_ARG, "trimul_contract_bwd: a, b, do_i, do_j, da and db are required");
  if (a.dtype != GNN_BF16 && a.dtype != GNN_F16)
    return set_error(GNN_ERR_UNSUPPORTED, "trimul_contract_bwd: 16-bit dtypes only");
  if (a.planes < 1 || a.N < 1) return set_error(GNN_ERR_ARG, "trimul_contract_bwd: planes and N must be positive");
  const void* ptr[6] = {a.a, a.b, a.do_i, a.do_j, a.da, a.db};
  for (const void* p : ptr)
    if (!aligned(p, 16)) return set_error(GNN_ERR_ARG, "trimul_contract_bwd: pointers must be 16-byte aligned");
  if (a.planes * ((a.N + 127) / 128) * ((a.N + 255) / 256) >= ((int64_t)1 << 31) || a.N >= ((int64_t)1 << 30))
    return set_error(GNN_ERR_UNSUPPORTED, "trimul_contract_bwd: grid too large");
  int rc = trimul_contract_bwd(a, (hipStream_t)stream);
  if (rc < 0) return rc;
  return hip_status((hipError_t)rc, "trimul_contract_bwd");
}

int gnn_trimul_relayout(const gnn_trimul_relayout_args* args, void* stream) {
  if (!args) return set_error(GNN_ERR_ARG, "trimul_relayout: args is NULL");
  const gnn_trimul_relayout_args& a = *args;
  if (!a.src || !a.dst) return set_error(GNN_ERR_ARG, "trimul_relayout: src and dst are required");
  if (a.dtype != GNN_BF16 && a.dtype != GNN_F16)
    return set_error(GNN_ERR_UNSUPPORTED, "trimul_relayout: 16-bit dtypes only");
  if (a.mode != GNN_RELAYOUT_PLANES_TO_PIXELS && a.mode != GNN_RELAYOUT_PIXELS_TO_BLOCKED)
    return set_error(GNN_ERR_ARG, "trimul_relayout: unknown mode");
  if (a.B < 1 || a.N < 1 || a.Ch < 1) return set_error(GNN_ERR_ARG, "trimul_relayout: B, N and Ch must be positive");
  if (a.Ch % 8 || a.src_ld % 8 || a.dst_ld % 8 || a.src_c0 % 8 || a.dst_c0 % 8 || a.src_c0 < 0 || a.dst_c0 < 0)
    return set_error(GNN_ERR_ARG, "trimul_relayout: Ch, row pitches and channel offsets must be multiples of 8");
  if (!aligned(a.src, 16) || !aligned(a.dst, 16))
    return set_error(GNN_ERR_ARG, "trimul_relayout: src and dst must be 16-byte aligned");
  const int64_t N8 = (a.N + 7) / 8 * 8;
  if (a.mode == GNN_RELAYOUT_PLANES_TO_PIXELS ? (a.src_ld < N8 || a.dst_c0 + a.Ch > a.dst_ld)
                                              : (a.src_c0 + a.Ch > a.src_ld))
    return set_error(GNN_ERR_ARG, "trimul_relayout: a row pitch is too small for its rows");
  int rc = trimul_relayout(a, (hipStream_t)stream);
  if (rc < 0) return rc;
  return hip_status((hipError_t)rc, "trimul_relayout");
}

const char* gnn_last_error(void) { return g_last_error.c_str(); }

const char* gnn_version(void) { return "0.1.0 gfx950"; }

}  // extern "C"
