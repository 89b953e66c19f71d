// extern "C" entry points declared in include/w4a8_amd.h.
//
// Every entry point validates its arguments on the host before launching and
// reports failures as a status code plus a per-thread message, the way the
// reference's host impls reject bad tensors with TORCH_CHECK before the launch
// (npu_ops/host/midgroup_w4a8_gemm.cpp:51-85, npu_ops/host/midgroup_quant_a.cpp:42-43).
// Nothing here allocates device memory or synchronises the stream.
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/w4a8_amd.h"
#include "kgeom.h"
#include "launch.h"

namespace w4a8 {

// Compute units of the current device, queried once per device (plans and
// workspace sizes follow it; a partitioned MI355X exposes fewer than 256).
// Without a usable device (the query fails, e.g. on a host without a GPU)
// the full part's 256 is assumed.
int device_cu_count() {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cached[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return 256;
    }
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        n = 256;
    }
    cached[dev].store(n, std::memory_order_relaxed);
    return n;
}

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, long long a = 0, long long b = 0, long long c = 0) {
    char buf[512];
    std::snprintf(buf, sizeof(buf), fmt, a, b, c);
    g_last_error = buf;
    return code;
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return W4A8_OK;
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return W4A8_ERR_HIP;
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Most rows one GEMM launch takes at row stride lda: the kernels address A
// with 32-bit offsets, up to 128 rows past a launch's last row, with 2^31
// added on top for out-of-range reads.  A multiple of 128 (the prefill tile)
// and at least 256, so that every chunk of a split call has more than 64 rows
// and stays on the prefill path (no workspace); 0 when not even that fits.
int64_t gemm_row_chunk(int64_t lda) {
    if (lda <= 0) return 0;
    const int64_t rows = ((1ll << 31) - 1) / lda - 128;
    const int64_t chunk = (rows / 128) * 128;
    return chunk >= 256 ? chunk : 0;
}

int check_problem(int64_t M, int64_t N, int64_t K, int64_t group) {
    if (M < 0 || N <= 0 || K <= 0 || group <= 0)
        return fail(W4A8_ERR_SHAPE, "bad shape: M=%lld N=%lld K=%lld (need M>=0, N>0, K>0)", M, N, K);
    if (M >= (1ll << 31) || N >= (1ll << 30) || K >= (1ll << 30) || group >= (1ll << 30))
        return fail(W4A8_ERR_SHAPE, "shape too large: M=%lld N=%lld K=%lld", M, N, K);
    return W4A8_OK;
}

int check_gemm(const void* a_q, int64_t lda, const void* a_scale, const void* w_tiles,
               const void* s_tiles, int scale_dtype, const void* y, int64_t ldy, int64_t M,
               int64_t N, int64_t K, int64_t group, const void* workspace,
               int64_t workspace_bytes, bool swiglu) {
    if (int rc = check_problem(M, N, K, group)) return rc;
    if (swiglu && N % 32 != 0)
        return fail(W4A8_ERR_UNSUPPORTED, "SwiGLU needs N/2 (N=%lld) to be a multiple of 16", N);
    if (scale_dtype != W4A8_DT_F16 && scale_dtype != W4A8_DT_BF16)
        return fail(W4A8_ERR_DTYPE, "scale_dtype %lld is neither F16 (0) nor BF16 (1)", scale_dtype);
    if (M == 0) return W4A8_OK;
    if (!a_q || !a_scale || !w_tiles || !s_tiles || !y) return fail(W4A8_ERR_NULL, "a required pointer is NULL");
    const int64_t kp = geom::kpad(K, group);
    const int64_t ncols = swiglu ? N / 2 : N;
    if (lda < kp || ldy < ncols)
        return fail(W4A8_ERR_SHAPE, "lda=%lld must be >= kpad=%lld and ldy=%lld >= the output width", lda, kp, ldy);
    if (lda % 16 != 0 || !aligned(a_q, 16))
        return fail(W4A8_ERR_ALIGN, "a_q must be 16-byte aligned with lda %% 16 == 0 (lda=%lld)", lda);
    // s_tiles: the wide decode layouts load the group scales of two columns
    // as one dword (gemm_wide.hip), so 4-byte alignment is part of the contract
    if (!aligned(w_tiles, 16) || !aligned(s_tiles, 4) || !aligned(y, 2) || !aligned(a_scale, 2))
        return fail(W4A8_ERR_ALIGN, "w_tiles must be 16-byte aligned, s_tiles 4-byte aligned; y, a_scale 2-byte aligned");
    // The kernels address the weight tiles with 32-bit buffer offsets,
    // including up to one tile past the end, and mark out-of-range reads with
    // an offset of 2^31 added on top (every path: the fused single-row linear too).
    const int64_t w_span = (geom::col_blocks(N) + 16) * geom::k_tiles(K, group) * geom::kTileBytes;
    if (w_span >= (1ll << 31))
        return fail(W4A8_ERR_UNSUPPORTED, "weights too large for 32-bit offsets (%lld B for N=%lld)", w_span, N);
    // A is addressed the same way: a call whose rows do not fit is split into
    // row chunks (run_gemm), which needs more than 64 rows and a chunk size.
    if (lda >= (1ll << 31) ||
        ((M + 128) * lda >= (1ll << 31) && (M <= kDecodeMaxM || gemm_row_chunk(lda) == 0)))
        return fail(W4A8_ERR_UNSUPPORTED, "M=%lld rows at lda=%lld exceed 32-bit activation offsets", M, lda);
    const int64_t need = w4a8_gemm_workspace_bytes(M, N, K, group);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned(workspace, 256)))
        return fail(W4A8_ERR_WORKSPACE, "workspace needs %lld bytes, 256-byte aligned (got %lld)", need,
                    workspace ? workspace_bytes : 0);
    return W4A8_OK;
}

int run_gemm(const void* a_q, int64_t lda, const void* a_scale, const void* w_tiles,
             const void* s_tiles, int scale_dtype, void* y, int64_t ldy, void* partials,
             int64_t M, int64_t N, int64_t K, int64_t group, void* workspace,
             int64_t workspace_bytes, void* stream, bool swiglu = false) {
    if (int rc = check_gemm(a_q, lda, a_scale, w_tiles, s_tiles, scale_dtype, y, ldy, M, N, K,
                            group, workspace, workspace_bytes, swiglu))
        return rc;
    if (M == 0) return W4A8_OK;
    GemmArgs a{};
    a.a_q = static_cast<const int8_t*>(a_q);
    a.lda = lda;
    a.a_scale = static_cast<const uint16_t*>(a_scale);
    a.w_tiles = static_cast<const uint8_t*>(w_tiles);
    a.s_tiles = static_cast<const uint16_t*>(s_tiles);
    a.scale_bf16 = scale_dtype == W4A8_DT_BF16;
    a.y = static_cast<uint16_t*>(y);
    a.ldy = ldy;
    a.partials = static_cast<int32_t*>(partials);
    a.swiglu = swiglu;
    a.M = M;
    a.N = N;
    a.K = K;
    a.group = group;
    a.workspace = workspace;
    a.workspace_bytes = workspace_bytes;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t chunk = gemm_row_chunk(lda);
    if ((M + 128) * lda < (1ll << 31)) {
        const hipError_t e = (M <= kDecodeMaxM) ? launch_gemm_decode(a, s) : launch_gemm_prefill(a, s);
        return hip_status(e, "w4a8_gemm launch");
    }
    // A too large for 32-bit offsets (e.g. K = 27648 past ~77k rows): the rows
    // go in balanced chunks of at most `chunk` (> 64 rows each: prefill
    // launches, no workspace).  The partial dump indexes rows of one launch.
    if (partials)
        return fail(W4A8_ERR_UNSUPPORTED, "M=%lld rows at lda=%lld need row chunks, not available with the "
                    "partial dump", M, lda);
    const int64_t nchunks = (M + chunk - 1) / chunk;
    for (int64_t c = 0; c < nchunks; ++c) {
        const int64_t m0 = (M * c) / nchunks, m1 = (M * (c + 1)) / nchunks;
        GemmArgs ac = a;
        ac.a_q = a.a_q + m0 * lda;
        ac.a_scale = a.a_scale + m0;
        ac.y = a.y + m0 * ldy;
        ac.M = m1 - m0;
        if (int rc = hip_status(launch_gemm_prefill(ac, s), "w4a8_gemm launch")) return rc;
    }
    return W4A8_OK;
}

// ---- scratch of the allocation-free GEMM (w4a8_gemm_noalloc)
// A file-scope device array: the runtime gives every GPU the library runs on
// its own copy, held until the process ends.  Host code must not pass the
// array's name to a kernel (on the host it is only a stand-in symbol): the
// device address of this GPU's copy comes from hipGetSymbolAddress, looked up
// once per device with that device current and kept.
static __device__ __align__(256) unsigned char scratch[W4A8_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// This device's copy of `scratch`, or a status code.
int scratch_for_current_device(void** out) {
    int dev = 0;
    if (int rc = hip_status(hipGetDevice(&dev), "w4a8_gemm_noalloc: hipGetDevice")) return rc;
    if (dev < 0 || dev >= kMaxScratchDevices)
        return fail(W4A8_ERR_UNSUPPORTED, "w4a8_gemm_noalloc: device %lld beyond the %lld supported", dev,
                    kMaxScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        if (int rc = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "w4a8_gemm_noalloc: hipGetSymbolAddress"))
            return rc;
        if (p == nullptr || !aligned(p, 256))
            return fail(W4A8_ERR_HIP, "w4a8_gemm_noalloc: scratch of device %lld is not 256-byte aligned", dev);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return W4A8_OK;
}

}  // namespace
}  // namespace w4a8

using namespace w4a8;

extern "C" {

int w4a8_abi_version(void) { return 10; }

const char* w4a8_last_error(void) { return g_last_error.c_str(); }

int w4a8_read_floor(const void* src, int64_t bytes, void* sink, void* stream) {
    if (bytes < 0 || bytes % 16 != 0) return fail(W4A8_ERR_SHAPE, "bytes=%lld must be a multiple of 16", bytes);
    if (bytes == 0) return W4A8_OK;
    if (!src || !sink) return fail(W4A8_ERR_NULL, "a required pointer is NULL");
    if (!aligned(src, 16) || !aligned(sink, 4)) return fail(W4A8_ERR_ALIGN, "src must be 16-byte, sink 4-byte aligned");
    if (bytes / 16 / 512 >= (1ll << 31)) return fail(W4A8_ERR_SHAPE, "bytes=%lld too large for one launch", bytes);
    return hip_status(launch_read_floor(src, bytes, static_cast<uint32_t*>(sink), static_cast<hipStream_t>(stream)),
                      "read_floor launch");
}

int w4a8_stream_capture_id(void* stream, unsigned long long* id) {
    if (id == nullptr) return fail(W4A8_ERR_NULL, "id is NULL");
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    if (int rc = hip_status(hipStreamGetCaptureInfo(static_cast<hipStream_t>(stream), &st, &cid),
                            "hipStreamGetCaptureInfo"))
        return rc;
    if (st != hipStreamCaptureStatusActive)
        return fail(W4A8_ERR_UNSUPPORTED, "stream is not being captured (capture status %lld)", static_cast<long long>(st));
    *id = cid;
    return W4A8_OK;
}

int w4a8_quant_act(const void* x, int64_t ldx, void* a_q, int64_t lda, void* a_scale, int64_t M,
                   int64_t K, int64_t group, void* stream) {
    if (M < 0 || K <= 0 || M >= (1ll << 31) || K >= (1ll << 30) || group < 0 || group >= (1ll << 30))
        return fail(W4A8_ERR_SHAPE, "bad shape: M=%lld K=%lld group=%lld", M, K, group);
    if (M == 0) return W4A8_OK;
    if (!x || !a_q || !a_scale) return fail(W4A8_ERR_NULL, "a required pointer is NULL");
    const int64_t width = group > 0 ? geom::kpad(K, group) : K;
    if (ldx < K || lda < width)
        return fail(W4A8_ERR_SHAPE, "ldx=%lld must be >= K and lda=%lld >= the output width %lld", ldx, lda, width);
    if (!aligned(x, 2) || !aligned(a_scale, 2)) return fail(W4A8_ERR_ALIGN, "x and a_scale must be 2-byte aligned");
    return hip_status(launch_quant_act(static_cast<const uint16_t*>(x), ldx, static_cast<int8_t*>(a_q), lda,
                                       static_cast<uint16_t*>(a_scale), M, K, group,
                                       static_cast<hipStream_t>(stream)),
                      "w4a8_quant_act launch");
}

int64_t w4a8_repacked_weight_bytes(int64_t N, int64_t K, int64_t group) {
    if (N <= 0 || K <= 0 || group <= 0) return -1;
    return geom::col_blocks(N) * geom::k_tiles(K, group) * geom::kTileBytes;
}

int64_t w4a8_repacked_scale_bytes(int64_t N, int64_t K, int64_t group) {
    if (N <= 0 || K <= 0 || group <= 0) return -1;
    return geom::col_blocks(N) * geom::num_groups(K, group) * 16 * 2;
}

int w4a8_repack(const void* w_q, const void* w_scale, int scale_dtype, void* w_tiles, void* s_tiles,
                int64_t N, int64_t K, int64_t group, void* stream) {
    if (int rc = check_problem(0, N, K, group)) return rc;
    if (scale_dtype != W4A8_DT_F16 && scale_dtype != W4A8_DT_BF16)
        return fail(W4A8_ERR_DTYPE, "scale_dtype %lld is neither F16 (0) nor BF16 (1)", scale_dtype);
    if (!w_q || !w_scale || !w_tiles || !s_tiles) return fail(W4A8_ERR_NULL, "a required pointer is NULL");
    if (!aligned(w_q, 4) || !aligned(w_tiles, 16) || !aligned(w_scale, 2) || !aligned(s_tiles, 2))
        return fail(W4A8_ERR_ALIGN, "w_q must be 4-byte, w_tiles 16-byte, scales 2-byte aligned");
    return hip_status(launch_repack(static_cast<const uint8_t*>(w_q), static_cast<const uint16_t*>(w_scale),
                                    static_cast<uint8_t*>(w_tiles), static_cast<uint16_t*>(s_tiles), N, K,
                                    group, static_cast<hipStream_t>(stream)),
                      "w4a8_repack launch");
}

int64_t w4a8_gemm_row_chunk(int64_t M, int64_t lda) {
    if (M <= 0 || lda <= 0) return 0;
    if ((M + 128) * lda < (1ll << 31)) return M;
    return M > kDecodeMaxM ? gemm_row_chunk(lda) : 0;
}

int64_t w4a8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group) {
    if (M <= 0 || N <= 0 || K <= 0 || group <= 0) return 0;
    return (M <= kDecodeMaxM) ? decode_workspace_bytes(M, N, K, group) : prefill_workspace_bytes(M, N, K, group);
}

int w4a8_gemm(const void* a_q, int64_t lda, const void* a_scale, const void* w_tiles, const void* s_tiles,
              int scale_dtype, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int64_t group,
              void* workspace, int64_t workspace_bytes, void* stream) {
    return run_gemm(a_q, lda, a_scale, w_tiles, s_tiles, scale_dtype, y, ldy, nullptr, M, N, K, group,
                    workspace, workspace_bytes, stream);
}

int w4a8_gemm_noalloc(const void* a_q, int64_t lda, const void* a_scale, const void* w_tiles, const void* s_tiles,
                      int scale_dtype, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int64_t group,
                      void* stream) {
    if (int rc = check_problem(M, N, K, group)) return rc;
    const int64_t need = w4a8_gemm_workspace_bytes(M, N, K, group);
    if (need > W4A8_NOALLOC_SCRATCH_BYTES)
        return fail(W4A8_ERR_WORKSPACE, "w4a8_gemm_noalloc: the shape needs %lld bytes of scratch, the static scratch "
                    "holds %lld (use w4a8_gemm with a workspace)", need, W4A8_NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    if (need > 0 && M > 0)
        if (int rc = scratch_for_current_device(&ws)) return rc;
    // the split sums need no clearing: the split GEMM writes every sum its reduce reads
    return run_gemm(a_q, lda, a_scale, w_tiles, s_tiles, scale_dtype, y, ldy, nullptr, M, N, K, group, ws,
                    ws ? W4A8_NOALLOC_SCRATCH_BYTES : 0, stream);
}

int w4a8_gemm_swiglu(const void* a_q, int64_t lda, const void* a_scale, const void* w_tiles,
                     const void* s_tiles, int scale_dtype, void* y, int64_t ldy, int64_t M, int64_t N,
                     int64_t K, int64_t group, void* workspace, int64_t workspace_bytes, void* stream) {
    return run_gemm(a_q, lda, a_scale, w_tiles, s_tiles, scale_dtype, y, ldy, nullptr, M, N, K, group,
                    workspace, workspace_bytes, stream, true);
}

int w4a8_linear(const void* x, int64_t ldx, const void* w_tiles, const void* s_tiles, int scale_dtype,
                void* y, int64_t ldy, void* a_q, int64_t lda, void* a_scale, int64_t M, int64_t N,
                int64_t K, int64_t group, void* workspace, int64_t workspace_bytes, void* stream) {
    if (int rc = check_gemm(a_q, lda, a_scale, w_tiles, s_tiles, scale_dtype, y, ldy, M, N, K, group, workspace,
                            workspace_bytes, false))
        return rc;
    if (M == 0) return W4A8_OK;
    if (!x) return fail(W4A8_ERR_NULL, "x is NULL");
    if (ldx < K) return fail(W4A8_ERR_SHAPE, "ldx=%lld must be >= K=%lld", ldx, K);
    if (!aligned(x, 2)) return fail(W4A8_ERR_ALIGN, "x must be 2-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    GemmArgs a{};
    a.a_q = static_cast<const int8_t*>(a_q);
    a.lda = lda;
    a.a_scale = static_cast<const uint16_t*>(a_scale);
    a.w_tiles = static_cast<const uint8_t*>(w_tiles);
    a.s_tiles = static_cast<const uint16_t*>(s_tiles);
    a.scale_bf16 = scale_dtype == W4A8_DT_BF16;
    a.y = static_cast<uint16_t*>(y);
    a.ldy = ldy;
    a.M = M;
    a.N = N;
    a.K = K;
    a.group = group;
    const auto* xb = static_cast<const uint16_t*>(x);
    if (linear_fusable(a, xb, ldx))
        return hip_status(launch_linear_fused(a, xb, ldx, static_cast<int8_t*>(a_q), lda, static_cast<uint16_t*>(a_scale), s),
                          "w4a8_linear launch");
    if (int rc = hip_status(launch_quant_act(xb, ldx, static_cast<int8_t*>(a_q), lda, static_cast<uint16_t*>(a_scale),
                                             M, K, group, s),
                            "w4a8_linear quant launch"))
        return rc;
    return run_gemm(a_q, lda, a_scale, w_tiles, s_tiles, scale_dtype, y, ldy, nullptr, M, N, K, group, workspace,
                    workspace_bytes, stream);
}

int w4a8_linear_fused(const void* x, int64_t ldx, int64_t M, int64_t N, int64_t K, int64_t group) {
    if (M <= 0 || N <= 0 || K <= 0 || group <= 0 || M >= (1ll << 31) || N >= (1ll << 30) || K >= (1ll << 30) ||
        group >= (1ll << 30))
        return 0;
    GemmArgs a{};
    a.M = M;
    a.N = N;
    a.K = K;
    a.group = group;
    return linear_fusable(a, static_cast<const uint16_t*>(x), ldx) ? 1 : 0;
}

int w4a8_gemm_debug_partials(const void* a_q, int64_t lda, const void* a_scale, const void* w_tiles,
                             const void* s_tiles, int scale_dtype, void* y, int64_t ldy, void* partials,
                             int64_t M, int64_t N, int64_t K, int64_t group, void* workspace,
                             int64_t workspace_bytes, void* stream) {
    if (!partials && M > 0) return fail(W4A8_ERR_NULL, "partials is NULL");
    if (partials && !aligned(partials, 4)) return fail(W4A8_ERR_ALIGN, "partials must be 4-byte aligned");
    return run_gemm(a_q, lda, a_scale, w_tiles, s_tiles, scale_dtype, y, ldy, partials, M, N, K, group,
                    workspace, workspace_bytes, stream);
}

int w4a8_midgroup_quant_a(const void* x, int64_t ldx, void* a_hi, void* a_lo, void* a_scale, void* a_ksum,
                          int64_t M, int64_t Mp, int64_t K, int64_t group, void* stream) {
    if (M < 0 || Mp < M || K <= 0 || group <= 0 || Mp >= (1ll << 31) || K >= (1ll << 30) || group >= (1ll << 30))
        return fail(W4A8_ERR_SHAPE, "bad shape: M=%lld Mp=%lld K=%lld (need 0 <= M <= Mp, K > 0)", M, Mp, K);
    if (Mp == 0) return W4A8_OK;
    if (!a_hi || !a_lo || !a_scale || !a_ksum || (M > 0 && !x)) return fail(W4A8_ERR_NULL, "a required pointer is NULL");
    if (M > 0 && ldx < K) return fail(W4A8_ERR_SHAPE, "ldx=%lld must be >= K=%lld", ldx, K);
    if (geom::num_groups(K, group) >= 65536)
        return fail(W4A8_ERR_UNSUPPORTED, "K=%lld group=%lld: more than 65535 groups", K, group);
    if ((M > 0 && !aligned(x, 2)) || !aligned(a_scale, 2) || !aligned(a_ksum, 4) || !aligned(a_hi, 4) ||
        !aligned(a_lo, 4))
        return fail(W4A8_ERR_ALIGN, "x/a_scale 2-byte, a_ksum/a_hi/a_lo 4-byte aligned");
    return hip_status(launch_quant_midgroup(static_cast<const uint16_t*>(x), ldx, static_cast<uint8_t*>(a_hi),
                                            static_cast<uint8_t*>(a_lo), static_cast<uint16_t*>(a_scale),
                                            static_cast<int32_t*>(a_ksum), M, Mp, K, group,
                                            static_cast<hipStream_t>(stream)),
                      "w4a8_midgroup_quant_a launch");
}

static int midgroup_gemm_impl(const void* a_hi, const void* a_lo, const void* a_scale, const void* a_ksum,
                              int64_t Ma, int64_t ld_as, const void* w_q, const void* w_scale, const void* w_zero,
                              void* y, int64_t ldy, void* partials, int64_t N, int64_t K, int64_t group,
                              void* workspace, int64_t workspace_bytes, void* stream, bool w_tiles = false) {
    if (int rc = check_problem(Ma, N, K, group)) return rc;
    if (geom::group_stride(group) % 128 != 0)
        return fail(W4A8_ERR_UNSUPPORTED, "group=%lld: the mid-group path needs ceil_to(group, 64) %% 128 == 0",
                    group);
    if (Ma == 0) return W4A8_OK;
    if (!a_hi || !a_lo || !a_scale || !a_ksum || !w_q || !w_scale || !y)
        return fail(W4A8_ERR_NULL, "a required pointer is NULL");
    if (ld_as < Ma || ldy < N) return fail(W4A8_ERR_SHAPE, "ld_as=%lld must be >= rows and ldy=%lld >= N", ld_as, ldy);
    if (!aligned(a_hi, 16) || !aligned(a_lo, 16) || !aligned(w_q, 16) || !aligned(a_scale, 2) ||
        !aligned(a_ksum, 4) || !aligned(w_scale, 2) || (w_zero && !aligned(w_zero, 2)) || !aligned(y, 2) ||
        (partials && !aligned(partials, 4)))
        return fail(W4A8_ERR_ALIGN, "planes and w_q 16-byte aligned; scales 2-, ksum and partials 4-byte aligned");
    const int64_t kb = geom::kpad(K, group) / 2;
    if ((Ma + 16) * kb >= (1ll << 31) || (N + 16) * kb >= (1ll << 31) ||
        (w_tiles && midgroup_tiles_bytes(N + 128, K, group) >= (1ll << 31)))
        return fail(W4A8_ERR_UNSUPPORTED, "operands too large for 32-bit offsets (%lld rows, N=%lld, %lld B/row)", Ma,
                    N, kb);
    // Prefill sizes with a workspace: the LDS-tiled prefill waves (no partial
    // dump there; dumps and calls without a workspace take the mid-group kernel)
    const int64_t need = partials ? 0 : midgroup_prefill_workspace_bytes(Ma, N, K, group);
    const bool prefill = need > 0 && workspace_bytes > 0;
    if (prefill) {
        if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
            return fail(W4A8_ERR_WORKSPACE, "workspace of %lld bytes (256-byte aligned) needed, got %lld", need,
                        workspace_bytes);
        if (geom::num_groups(K, group) * ld_as * 4 >= (1ll << 31))
            return fail(W4A8_ERR_UNSUPPORTED, "ld_as=%lld: activation ksums too large for 32-bit offsets", ld_as);
    } else if (midgroup_lds_bytes(Ma, K, group) > midgroup_lds_max()) {
        return fail(W4A8_ERR_UNSUPPORTED, "K=%lld group=%lld: too many groups for the staged scales (%lld B LDS)", K,
                    group, midgroup_lds_bytes(Ma, K, group));
    }
    MidgroupArgs a{};
    a.a_hi = a_hi;
    a.a_lo = a_lo;
    a.a_scale = a_scale;
    a.a_ksum = a_ksum;
    a.Ma = Ma;
    a.ld_as = ld_as;
    a.w_q = w_q;
    a.w_scale = w_scale;
    a.w_zero = w_zero;
    a.y = y;
    a.ldy = ldy;
    a.partials = partials;
    a.N = N;
    a.K = K;
    a.group = group;
    a.w_tiles = w_tiles;
    if (prefill)
        return hip_status(launch_gemm_midgroup_prefill(a, workspace, workspace_bytes, static_cast<hipStream_t>(stream)),
                          "w4a8_midgroup_gemm_ws launch");
    return hip_status(launch_gemm_midgroup(a, static_cast<hipStream_t>(stream)), "w4a8_midgroup_gemm launch");
}

int w4a8_midgroup_gemm(const void* a_hi, const void* a_lo, const void* a_scale, const void* a_ksum, int64_t Ma,
                       int64_t ld_as, const void* w_q, const void* w_scale, const void* w_zero, void* y, int64_t ldy,
                       void* partials, int64_t N, int64_t K, int64_t group, void* stream) {
    return midgroup_gemm_impl(a_hi, a_lo, a_scale, a_ksum, Ma, ld_as, w_q, w_scale, w_zero, y, ldy, partials, N, K,
                              group, nullptr, 0, stream);
}

int64_t w4a8_midgroup_gemm_workspace_bytes(int64_t Ma, int64_t N, int64_t K, int64_t group) {
    if (Ma < 0 || N <= 0 || K <= 0 || group <= 0) return 0;
    return midgroup_prefill_workspace_bytes(Ma, N, K, group);
}

int64_t w4a8_midgroup_tiles_bytes(int64_t N, int64_t K, int64_t group) {
    if (N <= 0 || K <= 0 || group <= 0) return -1;
    return midgroup_tiles_bytes(N, K, group);
}

int w4a8_midgroup_tile_weights(const void* w_q, void* w_tiles, int64_t N, int64_t K, int64_t group, void* stream) {
    if (int rc = check_problem(1, N, K, group)) return rc;
    if (!w_q || !w_tiles) return fail(W4A8_ERR_NULL, "w_q and w_tiles must not be NULL");
    if (!aligned(w_q, 16) || !aligned(w_tiles, 16)) return fail(W4A8_ERR_ALIGN, "w_q and w_tiles 16-byte aligned");
    return hip_status(launch_midgroup_tile(w_q, w_tiles, N, K, group, static_cast<hipStream_t>(stream)),
                      "w4a8_midgroup_tile_weights launch");
}

int w4a8_midgroup_gemm_tiled(const void* a_hi, const void* a_lo, const void* a_scale, const void* a_ksum, int64_t Ma,
                             int64_t ld_as, const void* w_tiles, const void* w_scale, const void* w_zero, void* y,
                             int64_t ldy, void* partials, int64_t N, int64_t K, int64_t group, void* workspace,
                             int64_t workspace_bytes, void* stream) {
    if (workspace_bytes < 0) return fail(W4A8_ERR_WORKSPACE, "workspace_bytes=%lld < 0", workspace_bytes);
    return midgroup_gemm_impl(a_hi, a_lo, a_scale, a_ksum, Ma, ld_as, w_tiles, w_scale, w_zero, y, ldy, partials, N,
                              K, group, workspace, workspace_bytes, stream, true);
}

int w4a8_midgroup_gemm_ws(const void* a_hi, const void* a_lo, const void* a_scale, const void* a_ksum, int64_t Ma,
                          int64_t ld_as, const void* w_q, const void* w_scale, const void* w_zero, void* y,
                          int64_t ldy, void* partials, int64_t N, int64_t K, int64_t group, void* workspace,
                          int64_t workspace_bytes, void* stream) {
    if (workspace_bytes < 0) return fail(W4A8_ERR_WORKSPACE, "workspace_bytes=%lld < 0", workspace_bytes);
    return midgroup_gemm_impl(a_hi, a_lo, a_scale, a_ksum, Ma, ld_as, w_q, w_scale, w_zero, y, ldy, partials, N, K,
                              group, workspace, workspace_bytes, stream);
}

int w4a8_rmsnorm_quant(const void* x, int64_t ldx, const void* residual, int64_t ldr, const void* weight, float eps,
                       void* sum_out, int64_t lds, void* h_out, int64_t ldh, void* a_q, int64_t lda, void* a_scale,
                       int64_t M, int64_t K, int64_t group, void* stream) {
    if (M < 0 || K <= 0 || M >= (1ll << 31) || group < 0)
        return fail(W4A8_ERR_SHAPE, "bad shape: M=%lld K=%lld group=%lld", M, K, group);
    if (K % 8 != 0 || K > 65536)
        return fail(W4A8_ERR_UNSUPPORTED, "K=%lld: the fused RMSNorm needs K %% 8 == 0 and K <= 65536", K);
    if (group > 0 && group % 8 != 0 && !geom::is_unpadded(K, group))
        return fail(W4A8_ERR_UNSUPPORTED, "group=%lld: a padded output layout needs group %% 8 == 0", group);
    if (!(eps >= 0.0f)) return fail(W4A8_ERR_SHAPE, "eps must be >= 0");
    if (M == 0) return W4A8_OK;
    if (!x || !weight || !a_q || !a_scale) return fail(W4A8_ERR_NULL, "a required pointer is NULL");
    const int64_t width = group > 0 ? geom::kpad(K, group) : K;
    if (ldx < K || lda < width || (residual && ldr < K) || (sum_out && lds < K) || (h_out && ldh < K))
        return fail(W4A8_ERR_SHAPE, "leading dimensions must cover the row (K=%lld, a_q width %lld)", K, width);
    auto al16 = [](const void* p, int64_t ld) { return !p || (aligned(p, 16) && ld % 8 == 0); };
    if (!al16(x, ldx) || !al16(residual, ldr) || !al16(sum_out, lds) || !al16(h_out, ldh) || !aligned(weight, 16) ||
        !aligned(a_q, 8) || lda % 8 != 0 || !aligned(a_scale, 2))
        return fail(W4A8_ERR_ALIGN, "bf16 rows 16-byte aligned (ld %% 8 == 0), a_q 8-byte aligned (lda %% 8 == 0)");
    RmsNormArgs a{};
    a.x = x;
    a.ldx = ldx;
    a.residual = residual;
    a.ldr = ldr;
    a.weight = weight;
    a.eps = eps;
    a.sum_out = sum_out;
    a.lds = lds;
    a.h_out = h_out;
    a.ldh = ldh;
    a.a_q = a_q;
    a.lda = lda;
    a.a_scale = a_scale;
    a.M = M;
    a.K = K;
    a.group = group;
    return hip_status(launch_rmsnorm_quant(a, static_cast<hipStream_t>(stream)), "w4a8_rmsnorm_quant launch");
}

int w4a8_rope_kv(const void* qkv, int64_t ldq, const void* bias, const void* cos_tab, const void* sin_tab, int64_t ldc,
                 int64_t L, const void* pos, void* q_out, void* k_cache, const int64_t* k_strides, void* v_cache,
                 const int64_t* v_strides, int64_t B, int64_t T, int64_t H, int64_t KVH, int64_t D, void* stream) {
    if (B < 0 || T < 0 || L <= 0 || B * T >= (1ll << 31))
        return fail(W4A8_ERR_SHAPE, "bad shape: B=%lld T=%lld L=%lld", B, T, L);
    if (H <= 0 || KVH <= 0 || D <= 0 || D % 2 != 0 || H + 2 * KVH > 65535 || (H + 2 * KVH) * D > (1ll << 30))
        return fail(W4A8_ERR_SHAPE, "bad heads: H=%lld KVH=%lld D=%lld (D even)", H, KVH, D);
    if (B * T == 0) return W4A8_OK;
    if (!qkv || !cos_tab || !sin_tab || !pos || !q_out || !k_cache || !v_cache || !k_strides || !v_strides)
        return fail(W4A8_ERR_NULL, "a required pointer is NULL");
    if (ldq < (H + 2 * KVH) * D || ldc < D / 2)
        return fail(W4A8_ERR_SHAPE, "leading dimensions must cover the row (qkv %lld, cos/sin %lld)",
                    (H + 2 * KVH) * D, D / 2);
    if (!aligned(qkv, 2) || !aligned(bias, 2) || !aligned(q_out, 2) || !aligned(k_cache, 2) || !aligned(v_cache, 2) ||
        !aligned(cos_tab, 4) || !aligned(sin_tab, 4) || !aligned(pos, 8))
        return fail(W4A8_ERR_ALIGN, "bf16 operands 2-byte, cos/sin 4-byte and pos 8-byte aligned");
    RopeKvArgs a{};
    a.qkv = static_cast<const uint16_t*>(qkv);
    a.ldq = ldq;
    a.bias = static_cast<const uint16_t*>(bias);
    a.cos = static_cast<const float*>(cos_tab);
    a.sin = static_cast<const float*>(sin_tab);
    a.ldc = ldc;
    a.pos = static_cast<const int64_t*>(pos);
    a.q_out = static_cast<uint16_t*>(q_out);
    a.k_cache = static_cast<uint16_t*>(k_cache);
    a.v_cache = static_cast<uint16_t*>(v_cache);
    for (int i = 0; i < 4; ++i) {
        if (k_strides[i] < 0 || v_strides[i] < 0) return fail(W4A8_ERR_SHAPE, "cache strides must be >= 0");
        a.ks[i] = k_strides[i];
        a.vs[i] = v_strides[i];
    }
    a.B = static_cast<int>(B);
    a.T = static_cast<int>(T);
    a.H = static_cast<int>(H);
    a.KVH = static_cast<int>(KVH);
    a.D = static_cast<int>(D);
    a.L = L;
    return hip_status(launch_rope_kv(a, static_cast<hipStream_t>(stream)), "w4a8_rope_kv launch");
}

int64_t w4a8_attention_chunks_per_split(int64_t B, int64_t H, int64_t KVH, int64_t Lc) {
    if (B <= 0 || H <= 0 || KVH <= 0 || H % KVH != 0 || Lc <= 0 || Lc % 64 != 0) return -1;
    // A single-token step has only B * KVH * ceil(G / 16) row tiles.  With at
    // least one per CU the cache is streamed unsplit (more splits only add
    // workspace traffic and the combine launch: measured on MI355X, 64 x 8 tiles
    // over 1280 positions 54 us unsplit against 63-86 us split 4-20 ways).
    // Fewer tiles are split until there is about one workgroup per CU, but
    // into at most max(8, chunks / 16) splits, the combine's sequential fold
    // being the price of each (one tile per KV head of one sequence: 10.6 us at
    // 7 splits against 13.9 us at 20).
    const int64_t nch = Lc / 64;
    const int64_t tiles = B * KVH * ((H / KVH + 15) / 16);
    const int64_t cus = device_cu_count();
    int64_t splits = 1;
    if (tiles < cus) splits = std::min({(cus + tiles - 1) / tiles, std::max<int64_t>(8, nch / 16), nch});
    return (nch + splits - 1) / splits;
}

int64_t w4a8_attention_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D, int64_t Lc, int64_t cps) {
    if (B <= 0 || T <= 0 || H <= 0 || D <= 0 || Lc <= 0 || Lc % 64 != 0 || cps <= 0) return -1;
    const int64_t ns = (Lc / 64 + cps - 1) / cps;
    return ns > 1 ? B * T * H * ns * (D + 4) * 4 : 0;
}

static int attention_impl(const void* q, const void* k_cache, const void* vt_cache, void* out, const void* pos,
                          int64_t B, int64_t T, int64_t H, int64_t KVH, int64_t D, int64_t L, int64_t Lc, int64_t cps,
                          float scale, void* workspace, int64_t ws_bytes, void* stream, const AttnArgs* rope) {
    if (B < 0 || T < 0 || B * T >= (1ll << 31))
        return fail(W4A8_ERR_SHAPE, "bad shape: B=%lld T=%lld", B, T);
    if (H <= 0 || KVH <= 0 || H % KVH != 0 || H / KVH > 65535 || H >= (1ll << 20))
        return fail(W4A8_ERR_SHAPE, "bad heads: H=%lld KVH=%lld (H a multiple of KVH)", H, KVH);
    if (D != 64 && D != 128) return fail(W4A8_ERR_UNSUPPORTED, "head_dim D=%lld: 64 or 128 supported", D);
    if (Lc <= 0 || Lc % 64 != 0 || L <= 0 || L > Lc || Lc * D * 2 >= (1ll << 31))
        return fail(W4A8_ERR_SHAPE, "cache: need 0 < L=%lld <= Lc=%lld, Lc a multiple of 64, Lc*D*2 < 2^31", L, Lc);
    if (cps <= 0 || cps > Lc / 64) return fail(W4A8_ERR_SHAPE, "chunks_per_split=%lld must be in [1, Lc/64]", cps);
    if (!std::isfinite(scale)) return fail(W4A8_ERR_SHAPE, "scale must be finite");
    if (B * T == 0) return W4A8_OK;
    if ((!q && !rope) || !k_cache || !vt_cache || !out || !pos) return fail(W4A8_ERR_NULL, "a required pointer is NULL");
    if (!aligned(q, 16) || !aligned(k_cache, 16) || !aligned(vt_cache, 16) || !aligned(out, 16) || !aligned(pos, 8) ||
        !aligned(workspace, 16))
        return fail(W4A8_ERR_ALIGN, "q, caches, out and workspace 16-byte aligned, pos 8-byte aligned");
    const int64_t pairs = B * KVH, G = H / KVH;
    const int64_t tiles = (G * T + 15) / 16;
    const int64_t ns = (Lc / 64 + cps - 1) / cps;
    const bool split = workspace != nullptr || rope != nullptr;   // the fused rotary path is a decode launch
    if (split) {
        const int64_t need = w4a8_attention_workspace_bytes(B, T, H, D, Lc, cps);
        if (ws_bytes < need) return fail(W4A8_ERR_WORKSPACE, "workspace needs %lld bytes (got %lld)", need, ws_bytes);
        if (pairs > 65535 || tiles > 65535 || pairs * G * T >= (1ll << 31))
            return fail(W4A8_ERR_UNSUPPORTED, "split launch: B*KVH=%lld and row tiles %lld must be <= 65535", pairs,
                        tiles);
    } else if (pairs * tiles >= (1ll << 31)) {
        return fail(W4A8_ERR_SHAPE, "too many row tiles: %lld", pairs * tiles);
    }
    AttnArgs a{};
    a.q = static_cast<const uint16_t*>(q);
    a.k = static_cast<const uint16_t*>(k_cache);
    a.vt = static_cast<const uint16_t*>(vt_cache);
    a.out = static_cast<uint16_t*>(out);
    a.ws = static_cast<float*>(workspace);
    a.pos = static_cast<const int64_t*>(pos);
    a.B = static_cast<int>(B);
    a.T = static_cast<int>(T);
    a.H = static_cast<int>(H);
    a.KVH = static_cast<int>(KVH);
    a.G = static_cast<int>(G);
    a.D = static_cast<int>(D);
    a.L = static_cast<int>(L);
    a.Lc = static_cast<int>(Lc);
    a.cps = static_cast<int>(cps);
    a.ns = static_cast<int>(ns);
    a.cs = static_cast<float>(1.4426950408889634 * static_cast<double>(scale));
    if (rope) {
        a.qkv = rope->qkv;
        a.ldq = rope->ldq;
        a.bias = rope->bias;
        a.cos = rope->cos;
        a.sin = rope->sin;
        a.ldc = rope->ldc;
        a.kw = static_cast<uint16_t*>(const_cast<void*>(k_cache));
        a.vtw = static_cast<uint16_t*>(const_cast<void*>(vt_cache));
    }
    return hip_status(launch_attention(a, split, static_cast<hipStream_t>(stream)), "w4a8_attention launch");
}

int w4a8_attention(const void* q, const void* k_cache, const void* vt_cache, void* out, const void* pos, int64_t B,
                   int64_t T, int64_t H, int64_t KVH, int64_t D, int64_t L, int64_t Lc, int64_t cps, float scale,
                   void* workspace, int64_t ws_bytes, void* stream) {
    return attention_impl(q, k_cache, vt_cache, out, pos, B, T, H, KVH, D, L, Lc, cps, scale, workspace, ws_bytes,
                          stream, nullptr);
}

int w4a8_attention_rope(const void* qkv, int64_t ldq, const void* bias, const void* cos_tab, const void* sin_tab,
                        int64_t ldc, void* k_cache, void* vt_cache, void* out, const void* pos, int64_t B, int64_t H,
                        int64_t KVH, int64_t D, int64_t L, int64_t Lc, int64_t cps, float scale, void* workspace,
                        int64_t ws_bytes, void* stream) {
    if (B > 0 && (!qkv || !cos_tab || !sin_tab)) return fail(W4A8_ERR_NULL, "a required pointer is NULL");
    if (KVH > 0 && H > 0 && D > 0 && (ldq < (H + 2 * KVH) * D || ldq % 8 != 0 || ldc < D / 2))
        return fail(W4A8_ERR_SHAPE, "qkv rows need ldq >= (H + 2 KVH) * D = %lld (a multiple of 8), cos/sin ldc >= D/2",
                    (H + 2 * KVH) * D);
    if (!aligned(qkv, 16) || !aligned(bias, 2) || !aligned(cos_tab, 4) || !aligned(sin_tab, 4))
        return fail(W4A8_ERR_ALIGN, "qkv 16-byte, bias 2-byte, cos/sin 4-byte aligned");
    AttnArgs r{};
    r.qkv = static_cast<const uint16_t*>(qkv);
    r.ldq = ldq;
    r.bias = static_cast<const uint16_t*>(bias);
    r.cos = static_cast<const float*>(cos_tab);
    r.sin = static_cast<const float*>(sin_tab);
    r.ldc = ldc;
    return attention_impl(nullptr, k_cache, vt_cache, out, pos, B, 1, H, KVH, D, L, Lc, cps, scale, workspace,
                          ws_bytes, stream, &r);
}

}  // extern "C"
