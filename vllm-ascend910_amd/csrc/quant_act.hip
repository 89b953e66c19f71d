// Dynamic per-token int8 activation quant (gfx950).
//
// Semantics follow the reference quantiser with a per-token spec
// (fakequant_lab/quant.py:89-105 group_params, :135-141 quantize_with):
//   s = bf16_rne(max|x| / 127)   -- fp32 divide, then rounded to bf16 BEFORE use
//   s = bf16 tiny (2^-126)       -- when that bf16 value is zero
//   q = clamp(rint(x / s), -128, 127), rint = round half to even, true fp32 divide
// The quotient is the IEEE divide's (the reference kernel insists on it,
// npu_ops/kernel/midgroup_quant_a.inc:55-62): a plain reciprocal multiply
// would flip half-way cases relative to torch.  The codes here come from a
// reciprocal multiply plus an exact half-way test (RowScale, common.h) that gives
// the divide's result for every input; rows whose scale is not a normal
// float divide per element.
//
// Layout: one workgroup per row (256 threads, 1024 for rows longer than 8192
// elements, so a decode-sized call still has enough loads in flight; long
// rows of a small batch are split into 1024-thread chunks).  The row is read
// once with 16-byte loads into registers, |x| is reduced as integers (for
// finite bf16 the magnitude order equals the order of the 15 low bits), then
// the same registers are quantised and written back as 8-byte int8 stores.
//
// Output order: plain (a_q[m, k]) or, for a ragged group geometry, the padded
// group layout the GEMM reads (kgeom.h; the reference's quantiser writes its
// activation planes in the same padded layout, midgroup_quant_a.inc:7-12):
// code k goes to (k / group) * stride + k % group, and the padding slots of
// every group are written as zero.
#include <type_traits>

#include "common.h"
#include "kgeom.h"
#include "launch.h"

namespace w4a8 {
namespace {

constexpr int kThreads = 256;

// Block-wide max of a uint32 over NT threads.
template <int NT>
__device__ __forceinline__ uint32_t block_max(uint32_t v, uint32_t* red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, 64)));
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    v = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) v = max(v, red[w]);
    return v;
}

// Padded group layout of one row.
struct PadMap {
    int group;    // quant group
    int stride;   // ceil_to(group, 64)
    int G;        // groups
    int kpad;     // padded row length
};

__device__ __forceinline__ int pad_dst(int k, const PadMap& pm) {
    const int g = k / pm.group;
    return g * pm.stride + (k - g * pm.group);
}

// Zero the padding slots [real, stride) of every group, in units of UNIT bytes
// (real lengths are multiples of UNIT).
template <int UNIT>
__device__ __forceinline__ void zero_pads(int8_t* qr, int K, const PadMap& pm) {
    for (int u = threadIdx.x; u < pm.kpad / UNIT; u += blockDim.x) {
        const int p = u * UNIT;
        const int g = p / pm.stride;
        const int real = (g + 1 < pm.G) ? pm.group : K - (pm.G - 1) * pm.group;
        if (p - g * pm.stride >= real) {
            if constexpr (UNIT == 8) *reinterpret_cast<uint2*>(qr + p) = make_uint2(0u, 0u);
            else qr[p] = 0;
        }
    }
}

// Vector path: K % 8 == 0, rows 16-byte aligned; with PAD also group % 8 == 0
// (an 8-code unit never straddles a group).  A workgroup quantises the
// 16-byte units [blockIdx.y * cv, +cv) of its row (at most VPT * NT), held in
// registers; with SPLIT (long rows of small batches, gridDim.y > 1) it also
// reads the rest of the row for the absmax, so each chunk's workgroup finds
// the same scale and the per-element work spreads over gridDim.y CUs.
template <int VPT, int NT, bool PAD, bool SPLIT>
__global__ __launch_bounds__(NT) void quant_act_vec_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int8_t* __restrict__ aq, int64_t lda,
    uint16_t* __restrict__ ascale, int K, const PadMap pm, int cv) {
    __shared__ uint32_t red[NT / 64];
    const int64_t row = blockIdx.x;
    const uint4* xr = reinterpret_cast<const uint4*>(x + row * ldx);
    const int nvec = K >> 3;
    const int v0 = SPLIT ? static_cast<int>(blockIdx.y) * cv : 0;
    const int v1 = SPLIT ? min(nvec, v0 + cv) : nvec;
    uint4 v[VPT];
    uint32_t amax = 0u;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = v0 + static_cast<int>(threadIdx.x) + i * NT;
        v[i] = (idx < v1) ? xr[idx] : make_uint4(0u, 0u, 0u, 0u);
        amax = max(amax, abs_bits_max8(v[i]));
    }
    if constexpr (SPLIT) {
#pragma unroll 4
        for (int idx = static_cast<int>(threadIdx.x); idx < nvec; idx += NT)
            if (idx < v0 || idx >= v1) amax = max(amax, abs_bits_max8(xr[idx]));
    }
    amax = block_max<NT>(amax, red);
    const uint32_t sbits = scale_from_amax(amax);
    const RowScale q = row_scale(bf16_bits_to_f32(sbits));
    const bool first = !SPLIT || blockIdx.y == 0;
    if (threadIdx.x == 0 && first) ascale[row] = static_cast<uint16_t>(sbits);
    int8_t* qr = aq + row * lda;
    // one uniform branch per row, not per element
    auto emit = [&](auto fast) __attribute__((always_inline)) {
        constexpr bool F = decltype(fast)::value;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int idx = v0 + static_cast<int>(threadIdx.x) + i * NT;
            if (idx < v1) {
                uint2 o;
                o.x = quant2<F>(v[i].x, q) | (quant2<F>(v[i].y, q) << 16);
                o.y = quant2<F>(v[i].z, q) | (quant2<F>(v[i].w, q) << 16);
                *reinterpret_cast<uint2*>(qr + (PAD ? pad_dst(idx * 8, pm) : idx * 8)) = o;
            }
        }
    };
    if (q.fast) emit(std::true_type{});
    else emit(std::false_type{});
    if constexpr (PAD) {
        if (first) zero_pads<8>(qr, K, pm);
    }
}

// General path: any K and strides; two passes over the row (the second one
// hits cache).
__global__ __launch_bounds__(kThreads) void quant_act_scalar_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int8_t* __restrict__ aq, int64_t lda,
    uint16_t* __restrict__ ascale, int K, bool pad, const PadMap pm) {
    __shared__ uint32_t red[4];
    const int64_t row = blockIdx.x;
    const uint16_t* xr = x + row * ldx;
    uint32_t amax = 0u;
    for (int k = threadIdx.x; k < K; k += kThreads) amax = max(amax, static_cast<uint32_t>(xr[k]) & 0x7fffu);
    amax = block_max<kThreads>(amax, red);
    const uint32_t sbits = scale_from_amax(amax);
    const RowScale q = row_scale(bf16_bits_to_f32(sbits));
    if (threadIdx.x == 0) ascale[row] = static_cast<uint16_t>(sbits);
    int8_t* qr = aq + row * lda;
    for (int k = threadIdx.x; k < K; k += kThreads)
        qr[pad ? pad_dst(k, pm) : k] = static_cast<int8_t>(quant_code<false>(bf16_bits_to_f32(xr[k]), q));
    if (pad) zero_pads<1>(qr, K, pm);
}

}  // namespace

hipError_t launch_quant_act(const uint16_t* x, int64_t ldx, int8_t* a_q, int64_t lda,
                            uint16_t* a_scale, int64_t M, int64_t K, int64_t group, hipStream_t stream) {
    if (M == 0) return hipSuccess;
    const dim3 grid(static_cast<unsigned>(M));
    const dim3 block(kThreads);
    const bool pad = group > 0 && !geom::is_unpadded(K, group);
    PadMap pm{};
    if (pad) {
        pm.group = static_cast<int>(group);
        pm.stride = static_cast<int>(geom::group_stride(group));
        pm.G = static_cast<int>(geom::num_groups(K, group));
        pm.kpad = static_cast<int>(geom::kpad(K, group));
    }
    const bool aligned = (K % 8 == 0) && (ldx % 8 == 0) && (lda % 8 == 0) && (!pad || group % 8 == 0) &&
                         (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(a_q) % 8 == 0);
    const int64_t nvec = K / 8;
    const int iK = static_cast<int>(K);
    const int cv = static_cast<int>(nvec);
    // Rows of up to 8192 elements: 256 threads.  Longer rows of a small batch
    // (M < 256, too few rows to fill the GPU): 1024-unit chunks, one 1024-
    // thread workgroup each; longer rows otherwise: 1024 threads per row.
    if (aligned && nvec > 4 * kThreads && M < 256) {
        const int chunks = static_cast<int>((nvec + 1023) / 1024);
        const dim3 g2(static_cast<unsigned>(M), static_cast<unsigned>(chunks));
        if (pad) quant_act_vec_kernel<1, 1024, true, true><<<g2, dim3(1024), 0, stream>>>(x, ldx, a_q, lda, a_scale, iK, pm, 1024);
        else quant_act_vec_kernel<1, 1024, false, true><<<g2, dim3(1024), 0, stream>>>(x, ldx, a_q, lda, a_scale, iK, pm, 1024);
        return hipGetLastError();
    }
    int vpt = 0;
    const bool wide = nvec > 4 * kThreads;
    const int nt = wide ? 4 * kThreads : kThreads;
    for (int v : {1, 2, 4, 8})
        if (vpt == 0 && aligned && nvec <= v * nt) vpt = v;
#define W4A8_QVEC(V, NT)                                                                                      \
    if (pad) quant_act_vec_kernel<V, NT, true, false><<<grid, dim3(NT), 0, stream>>>(x, ldx, a_q, lda, a_scale, iK, pm, cv); \
    else quant_act_vec_kernel<V, NT, false, false><<<grid, dim3(NT), 0, stream>>>(x, ldx, a_q, lda, a_scale, iK, pm, cv);
    if (vpt == 0) {
        quant_act_scalar_kernel<<<grid, block, 0, stream>>>(x, ldx, a_q, lda, a_scale, iK, pad, pm);
    } else if (!wide) {
        if (vpt == 1) { W4A8_QVEC(1, kThreads) }
        else if (vpt == 2) { W4A8_QVEC(2, kThreads) }
        else { W4A8_QVEC(4, kThreads) }
    } else {
        if (vpt == 1) { W4A8_QVEC(1, 4 * kThreads) }
        else if (vpt == 2) { W4A8_QVEC(2, 4 * kThreads) }
        else if (vpt == 4) { W4A8_QVEC(4, 4 * kThreads) }
        else { W4A8_QVEC(8, 4 * kThreads) }
    }
#undef W4A8_QVEC
    return hipGetLastError();
}

}  // namespace w4a8
