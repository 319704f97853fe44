// Host-side declarations shared by the kernel translation units and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>

#include "gnn_triangle.h"

namespace gnn {

// Records `msg` as this thread's last error and returns `code`.
int set_error(int code, const char* msg);

// Resident workgroups of a persistent kernel on the current device: occupancy x CU count,
// at least 1.
int persistent_grid(const void* fn, int threads, size_t smem);

int triattn_fwd(const gnn_triattn_args& a, hipStream_t stream);
int triattn_bwd(const gnn_triattn_bwd_args& a, hipStream_t stream);

// Row-resident attention (16-bit inputs, head dim <= 32, bounded N_res): the whole row of
// K and V staged in LDS, no barrier in the key loop.
bool triattn_row_applicable(const gnn_triattn_args& a);
size_t triattn_row_workspace_bytes(const gnn_triattn_args& a);

// The attention forward with its scratch in a static device array (no allocation anywhere).
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)16 << 20;
int triattn_fwd_noalloc(const gnn_triattn_args& a, hipStream_t stream);
int triattn_row_fwd(const gnn_triattn_args& a, hipStream_t stream);

// Row-resident attention backward for dq (with Delta) and dk / dv (16-bit inputs, head dim 32,
// bounded N_res); the pair-bias gradient stays with the tiled backward's dbias kernel.
bool triattn_bwd_row_applicable(const gnn_triattn_bwd_args& a);
int triattn_bwd_row_dq_dkdv(const gnn_triattn_bwd_args& a, hipStream_t stream);

// Workspace layout shared by the three trimul stages (byte offsets, see the C header).
struct TrimulLayout {
  size_t off_a, off_b, off_g, off_o, total;
};
TrimulLayout trimul_layout(int64_t B, int64_t N, int64_t C, int64_t Ch, int32_t dtype);

int trimul_proj(const gnn_trimul_args& a, hipStream_t stream);
int trimul_contract(const gnn_trimul_args& a, hipStream_t stream);
int trimul_out(const gnn_trimul_args& a, hipStream_t stream);

int pair_bias_proj(const gnn_pair_bias_args& a, hipStream_t stream);
int apb_gate_out(const gnn_apb_gate_out_args& a, hipStream_t stream);

// Backward helpers of the triangle multiplicative update.
int64_t layernorm_partials(int64_t rows, int64_t K);
int layernorm_rows(const gnn_layernorm_args& a, hipStream_t stream);
int64_t gate_bwd_partials(int64_t rows, int64_t K);
int gate_bwd(const gnn_gate_bwd_args& a, hipStream_t stream);
int64_t trimul_proj_bwd_partials(int64_t rows);
int64_t trimul_out_bwd_partials(int64_t B, int64_t N);
int trimul_out_bwd(const gnn_trimul_out_bwd_args& a, hipStream_t stream);
int trimul_proj_bwd(const gnn_trimul_proj_bwd_args& a, hipStream_t stream);
int trimul_contract_bwd(const gnn_trimul_contract_bwd_args& a, hipStream_t stream);
int trimul_relayout(const gnn_trimul_relayout_args& a, hipStream_t stream);

}  // namespace gnn
