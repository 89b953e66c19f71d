/*
 * w4a8_amd.h -- C ABI of the MI355X (gfx950) W4A8 per-group linear.
 *
 * This is the drop-in boundary for the reference's W4A8 dynamic linear
 * (GongCheng1919/vllm-ascend910).  The reference binds its device kernels
 * through torch.library C++ host impls; here the kernels sit behind plain
 * extern "C" entry points (raw device pointers, int64 sizes, a HIP stream
 * passed as void*), and the Python torch.library layer calls them through
 * ctypes.  Nothing here allocates device memory: outputs and workspace are
 * passed in by the caller, and every call is asynchronous on `stream`.
 *
 * Numeric contract (reference fakequant_lab/quant.py:89-141,
 * fakequant_lab/fake_linear.py:155-179):
 *   a_scale[m] = bf16_rne(max_k |x[m,k]| / 127), or bf16 tiny (2^-126) if 0
 *   a_q[m,k]   = clamp(round_half_even(x[m,k] / a_scale[m]), -128, 127)
 *   P_g[m,n]   = sum_{k in group g} a_q[m,k] * w_q[n,k]            (int32, exact)
 *   y[m,n]     = bf16_rne( a_scale[m] * sum_g P_g[m,n] * w_scale[g,n] )  (fp32)
 *
 * Status codes: every entry point returns 0 on success or one of the
 * W4A8_ERR_* codes; w4a8_last_error() returns a message for the calling
 * thread's most recent failure.  Invalid arguments are rejected before any
 * launch.
 */
#ifndef W4A8_AMD_H
#define W4A8_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum w4a8_status {
    W4A8_OK = 0,
    W4A8_ERR_NULL = 1,        /* a required pointer is NULL */
    W4A8_ERR_SHAPE = 2,       /* sizes are inconsistent or out of range */
    W4A8_ERR_DTYPE = 3,       /* unknown dtype code */
    W4A8_ERR_ALIGN = 4,       /* pointer / leading dimension alignment */
    W4A8_ERR_UNSUPPORTED = 5, /* valid per the reference, not built here yet */
    W4A8_ERR_WORKSPACE = 6,   /* workspace too small */
    W4A8_ERR_HIP = 7          /* the HIP runtime reported an error */
};

/* Scale dtype codes. */
enum w4a8_dtype { W4A8_DT_F16 = 0, W4A8_DT_BF16 = 1 };

/* Library ABI version (bumped on any signature or contract change: 4 = the
 * first build whose GEMM asks a workspace of some decode shapes; 5 adds
 * w4a8_rope_kv; 6 adds w4a8_stream_capture_id and requires 4-byte aligned
 * s_tiles; 7 adds w4a8_attention and its two size queries; 8 adds
 * w4a8_attention_rope; 9 adds w4a8_midgroup_gemm_ws and its size query; 10
 * adds w4a8_midgroup_tile_weights, w4a8_midgroup_tiles_bytes and
 * w4a8_midgroup_gemm_tiled). */
int w4a8_abi_version(void);

/* Message for the calling thread's last failed call ("" if none). */
const char* w4a8_last_error(void);

/*
 * The capture sequence id of a stream that is being captured into a HIP graph
 * (hipStreamGetCaptureInfo of the HIP runtime this library is bound to, which
 * is the one the process loaded): W4A8_OK and *id, or W4A8_ERR_UNSUPPORTED when
 * the stream is not capturing.  No counterpart in the reference; for callers
 * that key per-capture GEMM workspaces (the torch layer does) without binding
 * the HIP runtime by a file name of their own.
 */
int w4a8_stream_capture_id(void* stream, unsigned long long* id);

/*
 * Measurement kernel (no counterpart in the reference): a plain streaming
 * read of [src, src + bytes), bytes % 16 == 0, src 16-byte aligned, sink a
 * 4-byte device word written only for one improbable fold of the data.  The
 * bench times it over the same cold weight rotation as the decode GEMMs, as
 * the read floor those GEMMs are compared with.
 */
int w4a8_read_floor(const void* src, int64_t bytes, void* sink, void* stream);

/*
 * Dynamic per-token int8 activation quant.
 *   x       bf16 [M, ldx]   (first K columns used)
 *   a_q     int8 [M, lda]   output: with group == 0 (or a geometry without
 *                           padding, kpad(K, group) == K) the first K columns
 *                           hold a_q[m, k]; otherwise the first kpad columns
 *                           hold the padded group layout the GEMM reads --
 *                           code k at (k / group) * ceil_to(group, 64) + k % group,
 *                           padding slots zero (npu_ops/kernel/mg_kgeom.h:47-129)
 *   a_scale bf16 [M]
 * Replaces the reference's activation quantiser, kernel
 * npu_ops/kernel/midgroup_quant_a.inc:112-410 bound by
 * npu_ops/host/midgroup_quant_a.cpp:40-78, in its per-token mode
 * (fakequant_lab/quant.py:153-173 with QuantSpec(8, None)); like it, the
 * output follows the padded K layout of the weight.  The reference's MSD planes
 * and per-group activation scales are not produced here.
 */
int w4a8_quant_act(const void* x, int64_t ldx, void* a_q, int64_t lda, void* a_scale,
                   int64_t M, int64_t K, int64_t group, void* stream);

/*
 * Sizes of the repacked (gfx950 MFMA operand order) weight and scale buffers.
 * Weight: ceil(N/16) * ceil(kpad/128) tiles of 1024 bytes.  Scale:
 * ceil(N/16) * ceil(K/group) * 16 entries of 2 bytes.
 */
int64_t w4a8_repacked_weight_bytes(int64_t N, int64_t K, int64_t group);
int64_t w4a8_repacked_scale_bytes(int64_t N, int64_t K, int64_t group);

/*
 * Offline repacker.
 *   w_q      int8 [N, kpad/2]  reference packed layout: two int4 per byte
 *            along K, even k in the low nibble, each group zero-padded to a
 *            multiple of 64 elements (npu_ops/python/w4a8_ops.py:142-148,
 *            :231-239; npu_ops/kernel/mg_kgeom.h:90-102)
 *   w_scale  fp16/bf16 [G, N] group-major (npu_ops/host/midgroup_w4a8_gemm.cpp:82-85)
 *   w_tiles  output, w4a8_repacked_weight_bytes() bytes
 *   s_tiles  output, w4a8_repacked_scale_bytes() bytes, same dtype as w_scale
 * The reference has no repacker: its kernel reads w_q as stored.
 */
int w4a8_repack(const void* w_q, const void* w_scale, int scale_dtype, void* w_tiles,
                void* s_tiles, int64_t N, int64_t K, int64_t group, void* stream);

/*
 * Workspace bytes the GEMM needs for (M, N, K, group) on the current device;
 * 0 when none.  Only decode shapes past 8 rows on narrow N (fewer than four
 * two-block column groups per compute unit: under 2047 column blocks of 16 on
 * a 256-CU MI355X) with long K (at least 128 tiles of 128) use one: their K
 * is split over workgroups whose fp32 sums, [splits, M, ceil(N/16)*16], a
 * second kernel adds in split order.  A caller passes at least the size this
 * function returns (NULL/0 for 0), 256-byte aligned; calls that overlap in
 * time need workspaces of their own.  Prefill does not split K.
 */
int64_t w4a8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group);

/*
 * Rows per launch when w4a8_gemm splits a call of M rows at row stride lda
 * into row chunks: M itself when one launch takes them all (the kernels
 * address A with 32-bit offsets), 0 when the call is refused instead (64 rows
 * or fewer at that stride, or a stride too large for even 256 rows).  No
 * counterpart in the reference, whose host path has no such limit at its
 * shapes; a query for callers and tests.
 */
int64_t w4a8_gemm_row_chunk(int64_t M, int64_t lda);

/*
 * The grouped W4A8 GEMM with fused scale epilogue.
 *   a_q      int8 [M, lda]      the padded group layout of w4a8_quant_act with
 *                               the same group (lda >= kpad, lda % 16 == 0);
 *                               padding slots may hold any value (they meet
 *                               zero weight codes)
 *   a_scale  bf16 [M]
 *   w_tiles, s_tiles            (from w4a8_repack; scale_dtype as repacked;
 *                               w_tiles 16-byte and s_tiles 4-byte aligned)
 *   y        bf16 [M, ldy]      output
 * Calls whose activations exceed 32-bit offsets ((M + 128) * lda >= 2^31) run
 * as several launches over row chunks (w4a8_gemm_row_chunk); the debug
 * partial dump refuses such calls.
 * Replaces the reference GEMM, kernel npu_ops/kernel/midgroup_w4a8_gemm.inc:491-1169
 * bound by npu_ops/host/midgroup_w4a8_gemm.cpp:45-140 (run_midgroup_w4a8_gemm),
 * for symmetric weights and per-token activation scales.
 */
int w4a8_gemm(const void* a_q, int64_t lda, const void* a_scale, const void* w_tiles,
              const void* s_tiles, int scale_dtype, void* y, int64_t ldy, int64_t M, int64_t N,
              int64_t K, int64_t group, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * w4a8_gemm without the workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference, whose host path allocates its
 * workspace per call (npu_ops/host/midgroup_w4a8_gemm.cpp:116-118).  The fp32
 * split sums of the shapes that split K over workgroups go to a static device
 * array of W4A8_NOALLOC_SCRATCH_BYTES per GPU (the library's, held until the
 * process ends; no hipMalloc, no hipFree, nothing cleared -- every sum is
 * written before it is read).  Shapes that need more (w4a8_gemm_workspace_bytes
 * above the limit) return W4A8_ERR_WORKSPACE without launching; every
 * QwQ-32B projection at M <= 64 fits.  All calls on one GPU share that array:
 * calls that overlap in time on one GPU (other streams, concurrent replays)
 * race and must be ordered by the caller.  Results equal w4a8_gemm's bit for bit.
 */
#define W4A8_NOALLOC_SCRATCH_BYTES (8ll << 20)
int w4a8_gemm_noalloc(const void* a_q, int64_t lda, const void* a_scale, const void* w_tiles,
                      const void* s_tiles, int scale_dtype, void* y, int64_t ldy, int64_t M, int64_t N,
                      int64_t K, int64_t group, void* stream);

/*
 * The same GEMM over a merged gate/up weight (N = 2*I output columns: gate
 * rows [0, I), up rows [I, 2I), as vLLM's merged gate_up projection stores
 * them) with the SwiGLU activation fused into its epilogue:
 *   y[m, n] = bf16( bf16(silu(g)) * u ),  g = bf16(gemm[m, n]), u = bf16(gemm[m, n + I])
 *   y        bf16 [M, ldy], ldy >= I;  I % 16 == 0
 * silu(g) = g / (1 + exp(-g)) in fp32.  This is the rounding sequence of
 * `F.silu(g) * u` on the bf16 GEMM output in the reference's decoder layer
 * (npu_ops/python/bench_decode_layer.py:78-81; the vendor op it calls in its
 * graph bench, torch_npu.npu_swiglu, npu_ops/python/bench_decode_graph.py:64),
 * and every gate/up column accumulates exactly as in w4a8_gemm.  Saves the
 * [M, 2I] intermediate and the activation kernel.
 */
int w4a8_gemm_swiglu(const void* a_q, int64_t lda, const void* a_scale, const void* w_tiles,
                     const void* s_tiles, int scale_dtype, void* y, int64_t ldy, int64_t M, int64_t N,
                     int64_t K, int64_t group, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The whole W4A8 dynamic linear: per-token quant of bf16 x, then the GEMM,
 *   x        bf16 [M, ldx], ldx >= K, 2-byte aligned
 *   a_q      int8 [M, lda], a_scale bf16 [M]   receive the quantised
 *            activations (as w4a8_quant_act with this group writes them)
 *   the other arguments as for w4a8_gemm.
 * Results are those of w4a8_quant_act followed by w4a8_gemm, bit for bit.
 * For a single row (M == 1) with an unpadded K (and x 16-byte aligned,
 * ldx % 8 == 0) whose K split fits the fused prologue, the quant runs inside
 * the GEMM kernel on the GEMM's own split, one launch instead of two.
 * Replaces the reference linear method's quant-then-GEMM pair
 * (npu_ops/python/midgroup_quant.py:163-177, apply: midgroup_quant_a then
 * midgroup_w4a8_gemm) for the per-token symmetric path.
 */
int w4a8_linear(const void* x, int64_t ldx, const void* w_tiles, const void* s_tiles, int scale_dtype,
                void* y, int64_t ldy, void* a_q, int64_t lda, void* a_scale, int64_t M, int64_t N,
                int64_t K, int64_t group, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * 1 when w4a8_linear with these arguments runs as one fused launch, 0 when it
 * runs the quant and GEMM kernels (no counterpart in the reference: a query
 * for tests and schedulers; x is only inspected for alignment).
 */
int w4a8_linear_fused(const void* x, int64_t ldx, int64_t M, int64_t N, int64_t K, int64_t group);

/*
 * Parity hook: the same GEMM, which also writes every per-group int32 partial
 *   partials int32 [G, M, N],  partials[g][m][n] = P_g[m,n]
 * from the production kernel's own accumulators.  The reference computes the
 * same quantity in fakequant_lab/fake_linear.py:175 (`partial`).
 */
int w4a8_gemm_debug_partials(const void* a_q, int64_t lda, const void* a_scale,
                             const void* w_tiles, const void* s_tiles, int scale_dtype, void* y,
                             int64_t ldy, void* partials, int64_t M, int64_t N, int64_t K,
                             int64_t group, void* workspace, int64_t workspace_bytes,
                             void* stream);

/*
 * RMSNorm fused with the per-token activation quant (the producer-side fusion
 * the reference ranked first for decode, whose quant launches are pure
 * overhead: MGCKPT/P4_E2E.md:1043).  Per row:
 *   s = bf16(x + residual)   (residual may be NULL: s = x)
 *   h = bf16( bf16(s * (1 / sqrt(mean(s^2) + eps))) * weight )
 *   a_q, a_scale = w4a8_quant_act of h with the same group (padded layout)
 * the reference decoder layer's `rms_norm` (npu_ops/python/bench_decode_layer.py:36-38)
 * on the residual stream it keeps (:69-79).  sum_out (s) and h_out (h) are
 * optional bf16 outputs.  K % 8 == 0, K <= 65536; bf16 rows 16-byte aligned.
 * No counterpart entry point in the reference, which runs these as separate
 * vendor kernels (npu_rms_norm, then midgroup_quant_a).
 */
int w4a8_rmsnorm_quant(const void* x, int64_t ldx, const void* residual, int64_t ldr, const void* weight, float eps,
                       void* sum_out, int64_t lds, void* h_out, int64_t ldh, void* a_q, int64_t lda, void* a_scale,
                       int64_t M, int64_t K, int64_t group, void* stream);

/*
 * Rotary embedding of the q and k heads of a fused qkv projection output,
 * fused with the KV-cache append, for the decoder forward that drives the
 * W4A8 linears (QwQ-32B: H = 40 q heads, KVH = 8 kv heads, D = 128).
 *   qkv      bf16 [B * T, ldq]   per token: H q heads, KVH k heads, KVH v heads, D each
 *   bias     bf16 [(H + 2 KVH) * D] or NULL: the projection bias, added first as
 *                                torch adds two bf16 tensors, x = bf16(x + bias)
 *   cos_tab, sin_tab  fp32 [L, ldc]   angle tables (columns 0 .. D/2-1 used)
 *   pos      int64 [1] (device)  the position of token 0, shared by all B
 *                                sequences; token t sits at pos[0] + t (read on
 *                                the device, so a captured decode step follows
 *                                it).  Per-sequence positions are not supported.
 *   q_out    bf16 [B * T, H, D]  rotated q
 *   k_cache  element (b, h, d, p) at k_strides . (b, h, d, p): rotated k written at p
 *   v_cache  element (b, h, p, d) at v_strides . (b, h, p, d): v copied at p
 * Rotate-half form with the rounding sequence torch evaluates on float
 * tensors: y[i] = bf16(fl(x1*c) - fl(x2*s)), y[i+D/2] = bf16(fl(x2*c) +
 * fl(x1*s)), no fused multiply-add.  A token whose position falls outside
 * [0, L) writes nothing to the caches and zeros to its q rows.  No
 * counterpart in the reference, whose decoder-layer bench appends k and v in
 * place without a rotary embedding (npu_ops/python/bench_decode_layer.py:57-73).
 */
int w4a8_rope_kv(const void* qkv, int64_t ldq, const void* bias, const void* cos_tab, const void* sin_tab, int64_t ldc,
                 int64_t L, const void* pos, void* q_out, void* k_cache, const int64_t* k_strides, void* v_cache,
                 const int64_t* v_strides, int64_t B, int64_t T, int64_t H, int64_t KVH, int64_t D, void* stream);

/*
 * Grouped-query attention of T query tokens per sequence over the KV cache,
 * the attention of the decoder forward around the W4A8 linears.  Replaces the
 * reference decoder layer's `F.scaled_dot_product_attention(q, k, v,
 * enable_gqa=True)` over its in-place KV cache
 * (npu_ops/python/bench_decode_layer.py:70-73), with the causal mask of a
 * prefill and the cache length of a captured decode step read on the device.
 *   q        bf16 [B, T, H, D]     (w4a8_rope_kv's q_out)
 *   k_cache  bf16 [B, KVH, Lc, D]  keys, position-major
 *   vt_cache bf16 [B, KVH, D, Lc]  values transposed (position fastest)
 *   out      bf16 [B, T, H, D]
 *   pos      int64 [1] (device)    token t attends to positions 0 .. pos[0] + t
 *                                  (clamped to [0, L)); query head h*G + g reads
 *                                  KV head h, G = H / KVH
 * D = 64 or 128; Lc a multiple of 64, L <= Lc.  Per query row: scores in fp32
 * times `scale`, softmax in base 2 over chunks of 64 positions with a running
 * maximum, the probabilities rounded to bf16 for the product with V (fp32
 * accumulation), chunks grouped into splits of `chunks_per_split` whose states
 * are combined in split order, output bf16(O / l).  With `workspace` NULL one
 * workgroup walks all splits of its rows (prefill); with a workspace of
 * w4a8_attention_workspace_bytes bytes each split runs in its own workgroup and
 * a second kernel combines them (decode).  Both return the same bits for the
 * same row, cache and chunks_per_split.
 */
int w4a8_attention(const void* q, const void* k_cache, const void* vt_cache, void* out, const void* pos, int64_t B,
                   int64_t T, int64_t H, int64_t KVH, int64_t D, int64_t L, int64_t Lc, int64_t chunks_per_split,
                   float scale, void* workspace, int64_t ws_bytes, void* stream);

/*
 * A decode step's attention (one query token per sequence, split launch) with
 * w4a8_rope_kv's work fused in: the q heads are taken from the qkv projection
 * output and rotated in the attention kernel, and the step's rotated k and raw v
 * (+ bias) are used for position pos[0] and appended to the caches there -- the
 * bits w4a8_rope_kv followed by w4a8_attention give, in one launch fewer.
 *   qkv      bf16 [B, ldq]  (H q heads, KVH k heads, KVH v heads of D; 16-byte aligned, ldq % 8 == 0)
 *   bias     bf16 [(H + 2 KVH) * D] or NULL
 *   cos_tab, sin_tab  fp32 [>= L, ldc]  angle tables (columns 0 .. D/2-1 used)
 *   k_cache, vt_cache, out, pos, ... as w4a8_attention (T = 1); the caches are written at pos[0]
 * A position outside [0, L) writes nothing and attends with a zero query, as
 * w4a8_rope_kv leaves it.  Replaces the reference layer's in-place KV append and
 * SDPA call (npu_ops/python/bench_decode_layer.py:70-73) for a decode step.
 */
int w4a8_attention_rope(const void* qkv, int64_t ldq, const void* bias, const void* cos_tab, const void* sin_tab,
                        int64_t ldc, void* k_cache, void* vt_cache, void* out, const void* pos, int64_t B, int64_t H,
                        int64_t KVH, int64_t D, int64_t L, int64_t Lc, int64_t chunks_per_split, float scale,
                        void* workspace, int64_t ws_bytes, void* stream);

/* chunks_per_split for a decode step of B sequences (-1 for a bad shape): no split
 * once B * KVH * ceil(G / 16) single-token row tiles give every CU one, otherwise
 * splits up to about one workgroup per CU, at most max(8, Lc / 1024) of them. */
int64_t w4a8_attention_chunks_per_split(int64_t B, int64_t H, int64_t KVH, int64_t Lc);

/* Workspace bytes of the split launch (0 with a single split, -1 for a bad shape). */
int64_t w4a8_attention_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D, int64_t Lc,
                                       int64_t chunks_per_split);

/*
 * ---- Reference-compat mid-group path ----
 * The reference's own op pair, on its own tensors, for callers that keep its
 * exported mid-group checkpoints: per (token, K-group) activation scales, MSD
 * activation planes and an asymmetric int4 weight with per-(group, channel)
 * zero points.  Groups follow npu_ops/kernel/mg_kgeom.h (the reference fixes
 * group = 1024).
 *
 * Mid-group activation quant.
 *   x        bf16  [M, ldx]        (first K columns used)
 *   a_hi     int8  [Mp, kpad/2]    packed int4, hi = q >> 4
 *   a_lo     int8  [Mp, kpad/2]    packed int4, lo nibble = (q & 15) ^ 8
 *   a_scale  bf16  [G, Mp]         s = bf16_rne(max_{k in g}|x| / 127), tiny if 0
 *   a_ksum   int32 [G, Mp]         -sum_{k in g} q
 * with q = clamp(rint(x / s), -128, 127) per group (fakequant_lab/quant.py:89-141),
 * so that q = 16*hi + lo + 8.  Rows [M, Mp) are written as scale tiny, q = 0,
 * ksum 0; padding slots of a short last group as q = 0.
 * Replaces npu_ops/kernel/midgroup_quant_a.inc:112-410 bound by
 * npu_ops/host/midgroup_quant_a.cpp:40-78 (run_midgroup_quant_a), whose caller
 * chooses Mp = ceil_to(M, 16 | 64 | 128) (TileMFor, :37).
 */
int w4a8_midgroup_quant_a(const void* x, int64_t ldx, void* a_hi, void* a_lo, void* a_scale, void* a_ksum,
                          int64_t M, int64_t Mp, int64_t K, int64_t group, void* stream);

/*
 * Mid-group W4A8 GEMM on the reference's tensors as stored:
 *   a_hi, a_lo, a_scale, a_ksum   from w4a8_midgroup_quant_a (Ma rows; a_scale
 *                                 and a_ksum [G, ld_as], ld_as >= Ma)
 *   w_q      int8  [N, kpad/2]    packed int4 codes
 *   w_scale  bf16  [G, N]
 *   w_zero   bf16  [G, N]         zero point in code units, or NULL (symmetric)
 *   y        bf16  [Ma, ldy]
 *   partials int32 [G, Ma, N]     optional: I_g = sum_{k in g} A*(W - wz), exact
 *   y[m,n] = bf16( sum_g (float(I_g[m,n]) * w_scale[g,n]) * a_scale[g,m] )
 * (the reference's CPU definition, int4_cube_lab/host/gemm_ref.cpp:199-240),
 * each product and sum rounded in that order and the groups added in order, so
 * y is bf16 of ReferenceMidGroupGemm's fp32 result bit for bit.  The
 * reference kernel's w_ksum input is not needed: the activation bytes are
 * rebuilt exactly from the two planes.  Needs ceil_to(group, 64) % 128 == 0
 * and at most about 330 groups (every group's row and column values are staged
 * in LDS; more is W4A8_ERR_UNSUPPORTED).
 * Replaces npu_ops/kernel/midgroup_w4a8_gemm.inc:491-1169 bound by
 * npu_ops/host/midgroup_w4a8_gemm.cpp:45-140 (run_midgroup_w4a8_gemm).
 */
int w4a8_midgroup_gemm(const void* a_hi, const void* a_lo, const void* a_scale, const void* a_ksum, int64_t Ma,
                       int64_t ld_as, const void* w_q, const void* w_scale, const void* w_zero, void* y, int64_t ldy,
                       void* partials, int64_t N, int64_t K, int64_t group, void* stream);

/*
 * The same GEMM with a caller-owned workspace, as the reference host allocates
 * its GEMM workspace per call (npu_ops/host/midgroup_w4a8_gemm.cpp:116-118).
 * Where w4a8_midgroup_gemm_workspace_bytes(Ma, N, K, group) is non-zero (more
 * than 16 rows whose 64 x 128 output tiles number at least half the CU count,
 * group stride ceil_to(group, 64) a multiple of 128 and at least 256, offsets
 * below 2^31) and no partials are asked for, a call with workspace_bytes > 0
 * rebuilds the activation bytes from the two planes into the workspace
 * (256-byte aligned, at least that many bytes; W4A8_ERR_WORKSPACE otherwise)
 * and runs the LDS-tiled prefill kernel on w_q as stored.  Every output is the
 * same fp32 fold in group order as ReferenceMidGroupGemm's.  Any other call
 * (workspace_bytes == 0, a partial dump, a shape the query gives 0) runs as
 * w4a8_midgroup_gemm.
 */
int64_t w4a8_midgroup_gemm_workspace_bytes(int64_t Ma, int64_t N, int64_t K, int64_t group);
int w4a8_midgroup_gemm_ws(const void* a_hi, const void* a_lo, const void* a_scale, const void* a_ksum, int64_t Ma,
                          int64_t ld_as, const void* w_q, const void* w_scale, const void* w_zero, void* y,
                          int64_t ldy, void* partials, int64_t N, int64_t K, int64_t group, void* workspace,
                          int64_t workspace_bytes, void* stream);

/*
 * The compat GEMM on a weight reordered once at load time.  The reference
 * reads w_q [N, kpad/2] as stored on every call (its op takes it so,
 * npu_ops/host/midgroup_w4a8_gemm.cpp:45-140); its vLLM method converts
 * checkpoint tensors once after loading (npu_ops/python/midgroup_quant.py:148-161),
 * and at that point w4a8_midgroup_tile_weights writes the same bytes into
 * 1 KB tiles of w4a8_midgroup_tiles_bytes(N, K, group) bytes,
 *   w_tiles[nb][kt][q][c][0..15] = w_q[16 nb + c][64 kt + 16 q .. +15]
 * (zero past N and past kpad/2), which every compat kernel reads in whole
 * tiles.  w4a8_midgroup_gemm_tiled takes w_tiles in place of w_q, otherwise
 * as w4a8_midgroup_gemm_ws (the same workspace query, an upper bound here:
 * no per-call repack), with the same outputs bit for bit.
 */
int64_t w4a8_midgroup_tiles_bytes(int64_t N, int64_t K, int64_t group);
int w4a8_midgroup_tile_weights(const void* w_q, void* w_tiles, int64_t N, int64_t K, int64_t group, void* stream);
int w4a8_midgroup_gemm_tiled(const void* a_hi, const void* a_lo, const void* a_scale, const void* a_ksum, int64_t Ma,
                             int64_t ld_as, const void* w_tiles, const void* w_scale, const void* w_zero, void* y,
                             int64_t ldy, void* partials, int64_t N, int64_t K, int64_t group, void* workspace,
                             int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* W4A8_AMD_H */
