// Declarations shared by the two quantized GEMM translation units:
// orc_gemm.hip (vector path for Q8_0 / Q4_0, dispatch, C ABI) and
// orc_mmq.hip (matrix-core path for Q4_K / Q6_K and mixed launches).
#pragma once
#include "orc_internal.hpp"

#include <hip/hip_ext.h>

namespace orc {

// One GEMM launch: up to three weight segments sharing the activations X.
struct QmvParams {
    const uint8_t* w[3];
    float* y[3];
    const float* bias[3];
    int rows[3];
    int n_seg;
    int n_rows;  // logical rows: sum of the segment rows, or 2 x (gate, up) pairs
    int units;   // units per row
    uint64_t row_bytes;
    const float* x;
    int ldx, ldy, n_tok, n_in;
    const float* norm_w;
    float eps;
    int epi;
    int n_groups;
    int hs;               // matrix-core windowed mode: units of a wave's range staged at a time
    int seg_type[3];      // matrix-core mixed launches: weight type of each segment
    uint64_t seg_rb[3];   // and its row bytes
    int tok_block;        // tokens per token block (blockIdx.y) of a launch; n_tok counts all blocks
    int late_w;           // vector path: first weight batch issued after the activations are staged
    int split_rows;       // vector mixed launches: logical rows of the leading Q4_K segments
};

// Kernel timing of one launch: start / stop events taken from its dispatch.
struct LaunchEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};

// Device properties set by gemm_device_init.
extern int g_n_cu;
extern size_t g_lds_max;

// k_mmq type parameter: Q4_K and Q6_K segments in one launch (a Q4_K_M
// layer's Q|K|V, whose attn_v is Q6_K).
constexpr int kMixK = 256;

// Matrix-core path (orc_mmq.hip): tokens per launch for this shape (0 if none
// fit), and one launch of at most that many tokens.
bool mmq_type(int type);
int mmq_max_tokens(int type, const QmvParams& p);
int mmq_launch(int type, const QmvParams& p, hipStream_t s, const LaunchEvents& ev);
// the same for launches whose wave ranges are staged in windows (orc_mmq_win.hip)
int mmq_launch_windowed(int type, const QmvParams& p, hipStream_t s, const LaunchEvents& ev);
// Prefill launches (orc_mmq.hip): calls of at least kPfMinTok tokens on one
// K-quant type run k_mmq_pf, all tokens in one launch.
constexpr int kPfMinTok = 256;
bool mmq_prefill(int type, const QmvParams& p);
int mmq_prefill_launch(int type, const QmvParams& p, hipStream_t s, const LaunchEvents& ev);

}  // namespace orc
