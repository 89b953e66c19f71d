// Internal launchers behind the C ABI.  Arguments are already validated by the
// entry points in abi.hip; each launcher only picks a kernel variant and grid.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a8 {

// group > 0 with a ragged geometry (kpad != K) writes the padded group layout.
hipError_t launch_quant_act(const uint16_t* x, int64_t ldx, int8_t* a_q, int64_t lda,
                            uint16_t* a_scale, int64_t M, int64_t K, int64_t group,
                            hipStream_t stream);

hipError_t launch_repack(const uint8_t* w_q, const uint16_t* w_scale, uint8_t* w_tiles,
                         uint16_t* s_tiles, int64_t N, int64_t K, int64_t group,
                         hipStream_t stream);
// The weight tiles alone (the compat GEMM's prefill path repacks w_q per call).
hipError_t launch_repack_weights(const uint8_t* w_q, uint8_t* w_tiles, int64_t N, int64_t K, int64_t group,
                                 hipStream_t stream);

// Problem description shared by the GEMM paths.
struct GemmArgs {
    const int8_t* a_q;
    int64_t lda;
    const uint16_t* a_scale;   // bf16 [M]
    const uint8_t* w_tiles;
    const uint16_t* s_tiles;
    bool scale_bf16;
    uint16_t* y;               // bf16 [M, ldy]
    int64_t ldy;
    int32_t* partials;         // optional int32 [G, M, N]
    bool swiglu;               // y[:, n] = silu(gemm[:, n]) * gemm[:, n + N/2], n < N/2
    int64_t M, N, K, group;
    void* workspace;
    int64_t workspace_bytes;
};

// Decode path (M <= kDecodeMaxM): weight-stream bound, split-K.
constexpr int64_t kDecodeMaxM = 64;

int64_t decode_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group);
hipError_t launch_gemm_decode(const GemmArgs& a, hipStream_t stream);

// Decode launch configuration: register-ring depth D (tiles in flight per
// wave), columns blocks per workgroup CPW, waves per workgroup KW (the K
// split).  ``decode_config`` is the shape heuristic launch_gemm_decode uses;
// launch_gemm_decode_cfg takes an explicit one (cfg.D/CPW must name a built
// variant, otherwise hipErrorInvalidValue).
struct DecodeConfig {
    int D;
    int CPW;
    int KW;
    int MT = 0;       // 16-row tiles per workgroup; 0 = all rows in one workgroup
    int WIDE = 0;     // a WideLayout: the LDS-shared-activation kernel (gemm_wide.hip); D/CPW/KW/MT unused
    int SPLITS = 1;   // WIDE: workgroups along K (fp32 sums in the workspace, reduced by a second kernel)
    int STAGE = 0;    // 1: staged activations and scales (M <= 8, MT = 1, D = 4, CPW 1 or 2)
    int PSPLIT = 0;   // > 0: launch_gemm_prefill_split with this many K splits (other fields: the fallback plan)
};
DecodeConfig decode_config(int64_t M, int64_t N, int64_t K, int64_t group);
hipError_t launch_gemm_decode_cfg(const GemmArgs& a, const DecodeConfig& cfg, hipStream_t stream);

// Decode GEMM with the activations shared through LDS by the four column
// waves of a workgroup (gemm_wide.hip).  Layouts: 16-row tiles x 16-column
// blocks per wave; the x2 layouts also build the SwiGLU epilogue.
enum WideLayout : int {
    kWideNone = 0,
    kWide1x2 = 1,   // up to 16 rows
    kWide2x2 = 2,   // up to 32 rows
    kWide4x2 = 3,   // up to 64 rows
    kWide1x1 = 4,
    kWide2x1 = 5,
    kWide4x1 = 6,
};
hipError_t launch_gemm_wide(const GemmArgs& a, int layout, int splits, hipStream_t stream);
bool wide_layout_pairs(int layout);
// Workspace of a call with `splits` K splits (0 for one split).
int64_t wide_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group, int splits);

// Fused per-token quant + decode GEMM for one row (unpadded K, x 16-byte
// aligned with ldx % 8 == 0, and the decode heuristic's 2-block, 4-deep plan,
// whose K split it keeps).  The workgroup of column group 0 also
// writes a_q / a_scale.  launch_linear_fused returns hipErrorInvalidValue when
// linear_fusable is false.
bool linear_fusable(const GemmArgs& a, const uint16_t* x, int64_t ldx);
hipError_t launch_linear_fused(const GemmArgs& a, const uint16_t* x, int64_t ldx, int8_t* a_q, int64_t lda,
                               uint16_t* a_scale, hipStream_t stream);

// Adds `splits` fp32 K-split sums R [splits, M, ldr] in split order, applies
// the token scale and rounds to bf16 (one: int32 sums of a single group, folded
// with the column scales S, optional partial dump P).
hipError_t launch_split_reduce(const float* R, int64_t ldr, const uint16_t* a_scale, uint16_t* Y, int64_t ldy, int M,
                               int N, int splits, bool one, bool sbf16, const uint16_t* S, int32_t* P,
                               hipStream_t stream);

// Prefill path (M > kDecodeMaxM): MFMA bound, LDS-tiled.
int64_t prefill_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group);
hipError_t launch_gemm_prefill(const GemmArgs& a, hipStream_t stream);
// The prefill GEMM with an explicit tile height (128 or 64 rows), and the
// height launch_gemm_prefill picks.
hipError_t launch_gemm_prefill_bm(const GemmArgs& a, int bm, hipStream_t stream);
int prefill_tile_rows(int64_t M, int64_t N, int64_t group, bool swiglu);
// Up to 64 rows at group stride 128 (no SwiGLU, no partial dump): one 64-row
// tile of the 128 x 32 wave prefill kernel with K split over `splits`
// workgroups, then wide_reduce_kernel (splits > 1).
int64_t prefill_split_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group, int splits);
hipError_t launch_gemm_prefill_split(const GemmArgs& a, int splits, hipStream_t stream);


// Mid-group compat path (the reference's midgroup_quant_a / midgroup_w4a8_gemm).
hipError_t launch_quant_midgroup(const uint16_t* x, int64_t ldx, uint8_t* a_hi, uint8_t* a_lo,
                                 uint16_t* a_scale, int32_t* a_ksum, int64_t M, int64_t Mp, int64_t K,
                                 int64_t group, hipStream_t stream);

struct MidgroupArgs {
    const void* a_hi;
    const void* a_lo;
    const void* a_scale;   // bf16 [G, ld_as]
    const void* a_ksum;    // int32 [G, ld_as]
    int64_t Ma, ld_as;
    const void* w_q;       // [N, kpad/2]
    const void* w_scale;   // bf16 [G, N]
    const void* w_zero;    // bf16 [G, N] or null (symmetric)
    void* y;
    int64_t ldy;
    void* partials;        // optional int32 [G, Ma, N]
    int64_t N, K, group;
    bool w_tiles;          // w_q in launch_midgroup_tile's layout instead of [N, kpad/2]
};
// Bytes of LDS the staged scales need for one workgroup of the smallest tile
// the rows take (16 rows up to 16 rows or where 64 rows' values do not fit),
// and the most a launch gets (shapes above it are refused).
int64_t midgroup_lds_bytes(int64_t Ma, int64_t K, int64_t group);
int64_t midgroup_lds_max();
hipError_t launch_gemm_midgroup(const MidgroupArgs& a, hipStream_t stream);
// The same GEMM at prefill sizes on gemm_prefill_kernel's LDS-tiled waves
// (gemm_prefill.hip): the activation planes rebuilt into a workspace of
// midgroup_prefill_workspace_bytes (0: the shape takes launch_gemm_midgroup;
// no partial dump).  Outputs equal a one-wave-per-column-tile walk of
// ReferenceMidGroupGemm's fold order.
int64_t midgroup_prefill_workspace_bytes(int64_t Ma, int64_t N, int64_t K, int64_t group);
// w_q [N, kpad/2] -> 1 KB tiles [ceil(N/16)][k_tiles][quad][column][16 bytes]
// (the same bytes; every compat kernel reads either layout).
int64_t midgroup_tiles_bytes(int64_t N, int64_t K, int64_t group);
hipError_t launch_midgroup_tile(const void* w_q, void* w_tiles, int64_t N, int64_t K, int64_t group,
                                hipStream_t stream);
hipError_t launch_gemm_midgroup_prefill(const MidgroupArgs& a, void* ws, int64_t ws_bytes, hipStream_t stream);

// RMSNorm (+ optional residual add) fused with the per-token quant.
struct RmsNormArgs {
    const void* x;
    int64_t ldx;
    const void* residual;   // optional
    int64_t ldr;
    const void* weight;     // bf16 [K]
    float eps;
    void* sum_out;          // optional bf16 [M, lds]
    int64_t lds;
    void* h_out;            // optional bf16 [M, ldh]
    int64_t ldh;
    void* a_q;
    int64_t lda;
    void* a_scale;
    int64_t M, K, group;
};
hipError_t launch_rmsnorm_quant(const RmsNormArgs& a, hipStream_t stream);

// Rotary embedding of the q and k heads of a fused qkv projection output and
// the KV-cache append (rope_kv.hip).
struct RopeKvArgs {
    const uint16_t* qkv;    // bf16 [B * T, ldq]: H q heads, KVH k heads, KVH v heads of D
    int64_t ldq;
    const uint16_t* bias;   // optional bf16 [(H + 2 KVH) * D], added before the rotation
    const float* cos;       // fp32 [L, ldc], columns 0 .. D/2-1 used
    const float* sin;
    int64_t ldc;
    const int64_t* pos;     // device: position of token 0 of every sequence
    uint16_t* q_out;        // bf16 [B * T, H, D]
    uint16_t* k_cache;      // element (b, h, d, p) at b*ks[0] + h*ks[1] + d*ks[2] + p*ks[3]
    int64_t ks[4];
    uint16_t* v_cache;      // element (b, h, p, d) at b*vs[0] + h*vs[1] + p*vs[2] + d*vs[3]
    int64_t vs[4];
    int B, T, H, KVH, D;
    int64_t L;              // cache positions
};
hipError_t launch_rope_kv(const RopeKvArgs& a, hipStream_t stream);

// Grouped-query attention of the query rows of a decode step or a prefill over
// the KV cache (attention.hip).
struct AttnArgs {
    const uint16_t* q;      // bf16 [B, T, H, D]
    const uint16_t* k;      // bf16 [B, KVH, Lc, D]
    const uint16_t* vt;     // bf16 [B, KVH, D, Lc]
    uint16_t* out;          // bf16 [B, T, H, D]
    float* ws;              // split launch with ns > 1: B * H * T * ns states of D + 4 floats
    const int64_t* pos;     // device: position of token 0 of every sequence
    int B, T, H, KVH, G, D; // G = H / KVH query heads per KV head; D = 64 or 128
    int L, Lc;              // attended positions are clamped to [0, L); Lc = cache axis, multiple of 64
    int cps, ns;            // chunks of 64 positions per split; splits = ceil(Lc / 64 / cps)
    float cs;               // log2(e) * softmax scale
    // Decode (T = 1) with the rotary embedding and the KV-cache append fused in
    // (qkv set; q unused): the q heads and the step's k and v come from the qkv
    // projection output, rotated as w4a8_rope_kv rotates them.
    const uint16_t* qkv;    // bf16 [B, ldq]: H q heads, KVH k heads, KVH v heads of D
    int64_t ldq;
    const uint16_t* bias;   // optional bf16 [(H + 2 KVH) * D], added before the rotation
    const float* cos;       // fp32 [>= L, ldc], columns 0 .. D/2-1 used
    const float* sin;
    int64_t ldc;
    uint16_t* kw;           // the caches (k, vt above), written at the step's position
    uint16_t* vtw;
};
hipError_t launch_attention(const AttnArgs& a, bool split, hipStream_t stream);

// Streaming read of [src, src + bytes) (bytes a multiple of 16, src 16-byte
// aligned); sink (4 bytes) is written only for one improbable fold value.
hipError_t launch_read_floor(const void* src, int64_t bytes, uint32_t* sink, hipStream_t stream);

int device_cu_count();

}  // namespace w4a8
