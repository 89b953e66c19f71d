// RMSNorm fused with the dynamic per-token int8 activation quant (gfx950).
//
// One pass per row of what the reference's decoder layer runs as separate
// kernels (npu_ops/python/bench_decode_layer.py:36-38 rms_norm, then the
// activation quant of the next projection):
//   s      = bf16(x + residual)            (optional fused residual add; s = x without one)
//   r      = 1 / sqrt(mean(float(s)^2) + eps)            fp32, IEEE sqrt and divide
//   h      = bf16( float(bf16(float(s) * r)) * float(w) )  the reference's two bf16 roundings
//   a_q, a_scale = per-token quant of h      (quant_act.hip semantics, quant.py:89-141)
// The sum of squares is one fixed tree over the row's 8-element units: each
// unit's squares are added in element order, then units u and u ^ 2^b are
// paired for b = 0, 1, 2, ... (units past the row add exact zeros).  The tree
// depends only on the unit index, not on how units are spread over threads,
// so a row's result does not depend on the launch shape the batch size
// selects; its order differs from torch's vectorised mean, which moves r by
// at most an fp32 ulp.  Optionally writes s
// (the updated residual stream) and h.  One workgroup per row, the row held in
// registers (256 threads up to 8192 elements -- one 8-element unit per thread
// for up to 64 rows -- and 1024 threads up to 65536).
#include <type_traits>

#include "common.h"
#include "kgeom.h"
#include "launch.h"

namespace w4a8 {
namespace {

constexpr uint32_t kTinyRN = 0x0080u;   // bf16 2^-126

struct RmsParams {
    const uint16_t* x;
    int64_t ldx;
    const uint16_t* res;   // optional
    int64_t ldr;
    const uint16_t* w;     // [K]
    float eps;
    uint16_t* sum_out;     // optional
    int64_t lds;
    uint16_t* h_out;       // optional
    int64_t ldh;
    int8_t* a_q;
    int64_t lda;
    uint16_t* a_scale;
    int K;
    int group, stride, G;  // padded output layout when group > 0
    bool pad;
};

__device__ __forceinline__ float bf16r(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

// Sum of the VPT per-unit partials v[i] of every thread, where thread t holds
// unit t + i NT: unit-index bits 0-5 are the lane (xor shuffles, bit 0 first),
// the next log2(NT / 64) bits the wave, the bits above the register index i
// -- so pairing lanes, then waves, then registers, each in increasing bit
// order, is the tree over the unit index, for every NT.
template <int VPT, int NT>
__device__ __forceinline__ float block_sum_units(float (&v)[VPT], float* red) {
    constexpr int NW = NT / 64;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) v[i] += __shfl_xor(v[i], off, 64);
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int i = 0; i < VPT; ++i) red[i * NW + (threadIdx.x >> 6)] = v[i];
    }
    __syncthreads();
    float r[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        float w[NW];
#pragma unroll
        for (int k = 0; k < NW; ++k) w[k] = red[i * NW + k];
#pragma unroll
        for (int st = 1; st < NW; st <<= 1)
#pragma unroll
            for (int k = 0; k + st < NW; k += 2 * st) w[k] += w[k + st];
        r[i] = w[0];
    }
#pragma unroll
    for (int st = 1; st < VPT; st <<= 1)
#pragma unroll
        for (int i = 0; i + st < VPT; i += 2 * st) r[i] += r[i + st];
    __syncthreads();
    return r[0];
}

template <int NT>
__device__ __forceinline__ uint32_t block_max_u(uint32_t v, uint32_t* red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, 64)));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t m = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) m = max(m, red[i]);
    return m;
}


// VPT units of 8 elements per thread; K % 8 == 0, rows 16-byte aligned.
template <int VPT, int NT, bool RES>
__global__ __launch_bounds__(NT) void rmsnorm_quant_kernel(const RmsParams p) {
    static_assert((VPT & (VPT - 1)) == 0 && (NT & (NT - 1)) == 0, "power-of-two units and threads");
    __shared__ float redf[VPT * NT / 64];
    __shared__ uint32_t redu[NT / 64];
    const int64_t row = blockIdx.x;
    const int nvec = p.K >> 3;
    const uint4* xr = reinterpret_cast<const uint4*>(p.x + row * p.ldx);
    const uint4* rr = RES ? reinterpret_cast<const uint4*>(p.res + row * p.ldr) : nullptr;
    const uint4* wr = reinterpret_cast<const uint4*>(p.w);

    // the norm weight is requested with the row (it is used after the
    // reduction, which would otherwise wait for a second memory round trip)
    uint4 wv[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = static_cast<int>(threadIdx.x) + i * NT;
        wv[i] = idx < nvec ? wr[idx] : make_uint4(0u, 0u, 0u, 0u);
    }
    // s = bf16(x + r) kept as packed bf16 pairs; per-thread sum of squares
    uint4 v[VPT];
    float ss[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = static_cast<int>(threadIdx.x) + i * NT;
        uint4 a = make_uint4(0u, 0u, 0u, 0u);
        if (idx < nvec) {
            a = xr[idx];
            if constexpr (RES) {
                const uint4 b = rr[idx];
                uint32_t* pa = reinterpret_cast<uint32_t*>(&a);
                const uint32_t* pb = reinterpret_cast<const uint32_t*>(&b);
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const uint32_t lo = f32_to_bf16_bits(__uint_as_float(pa[d] << 16) + __uint_as_float(pb[d] << 16));
                    const uint32_t hi = f32_to_bf16_bits(__uint_as_float(pa[d] & 0xffff0000u) +
                                                         __uint_as_float(pb[d] & 0xffff0000u));
                    pa[d] = lo | (hi << 16);
                }
            }
        }
        v[i] = a;
        const uint32_t* pa = reinterpret_cast<const uint32_t*>(&v[i]);
        ss[i] = 0.0f;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const float e0 = __uint_as_float(pa[d] << 16), e1 = __uint_as_float(pa[d] & 0xffff0000u);
            ss[i] = fmaf(e0, e0, ss[i]);
            ss[i] = fmaf(e1, e1, ss[i]);
        }
    }
    const float tot = block_sum_units<VPT, NT>(ss, redf);
    const float r = 1.0f / sqrtf(tot / static_cast<float>(p.K) + p.eps);

    // h = bf16(bf16(s * r) * w); absmax of h
    uint32_t amax = 0u;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = static_cast<int>(threadIdx.x) + i * NT;
        if (idx >= nvec) continue;
        if (p.sum_out) *reinterpret_cast<uint4*>(p.sum_out + row * p.lds + idx * 8) = v[i];
        uint32_t* pa = reinterpret_cast<uint32_t*>(&v[i]);
        const uint32_t* pw = reinterpret_cast<const uint32_t*>(&wv[i]);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const float h0 = bf16r(bf16r(__uint_as_float(pa[d] << 16) * r) * __uint_as_float(pw[d] << 16));
            const float h1 = bf16r(bf16r(__uint_as_float(pa[d] & 0xffff0000u) * r) *
                                   __uint_as_float(pw[d] & 0xffff0000u));
            pa[d] = (__float_as_uint(h0) >> 16) | (__float_as_uint(h1) & 0xffff0000u);
            amax = max(amax, max(pa[d] & 0x7fffu, (pa[d] >> 16) & 0x7fffu));
        }
        if (p.h_out) *reinterpret_cast<uint4*>(p.h_out + row * p.ldh + idx * 8) = v[i];
    }
    amax = block_max_u<NT>(amax, redu);
    uint32_t sbits = f32_to_bf16_bits(bf16_bits_to_f32(amax) / 127.0f);
    if ((sbits & 0x7fffu) == 0u) sbits = kTinyRN;
    const RowScale sc = row_scale(bf16_bits_to_f32(sbits));
    if (threadIdx.x == 0) p.a_scale[row] = static_cast<uint16_t>(sbits);
    int8_t* qr = p.a_q + row * p.lda;
    // one uniform branch per row between the reciprocal and divide paths
    auto emit = [&](auto fast) __attribute__((always_inline)) {
        constexpr bool F = decltype(fast)::value;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int idx = static_cast<int>(threadIdx.x) + i * NT;
            if (idx >= nvec) continue;
            const uint32_t* pa = reinterpret_cast<const uint32_t*>(&v[i]);
            uint2 o;
            uint32_t wd[2] = {0u, 0u};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const int q0 = quant_code<F>(__uint_as_float(pa[d] << 16), sc);
                const int q1 = quant_code<F>(__uint_as_float(pa[d] & 0xffff0000u), sc);
                wd[d >> 1] |= ((static_cast<uint32_t>(q0) & 0xffu) | ((static_cast<uint32_t>(q1) & 0xffu) << 8))
                              << (16 * (d & 1));
            }
            o.x = wd[0];
            o.y = wd[1];
            int k0 = idx * 8;
            if (p.pad) {
                const int g = k0 / p.group;
                k0 = g * p.stride + (k0 - g * p.group);
            }
            *reinterpret_cast<uint2*>(qr + k0) = o;
        }
    };
    if (sc.fast) emit(std::true_type{});
    else emit(std::false_type{});
    if (p.pad) {
        // zero the padding slots (real lengths are multiples of 8 here)
        const int kp = static_cast<int>(geom::kpad(p.K, p.group));
        for (int u = threadIdx.x; u < kp / 8; u += NT) {
            const int q = u * 8, g = q / p.stride;
            const int real = (g + 1 < p.G) ? p.group : p.K - (p.G - 1) * p.group;
            if (q - g * p.stride >= real) *reinterpret_cast<uint2*>(qr + q) = make_uint2(0u, 0u);
        }
    }
}

}  // namespace

hipError_t launch_rmsnorm_quant(const RmsNormArgs& a, hipStream_t stream) {
    if (a.M == 0) return hipSuccess;
    RmsParams p{};
    p.x = static_cast<const uint16_t*>(a.x);
    p.ldx = a.ldx;
    p.res = static_cast<const uint16_t*>(a.residual);
    p.ldr = a.ldr;
    p.w = static_cast<const uint16_t*>(a.weight);
    p.eps = a.eps;
    p.sum_out = static_cast<uint16_t*>(a.sum_out);
    p.lds = a.lds;
    p.h_out = static_cast<uint16_t*>(a.h_out);
    p.ldh = a.ldh;
    p.a_q = static_cast<int8_t*>(a.a_q);
    p.lda = a.lda;
    p.a_scale = static_cast<uint16_t*>(a.a_scale);
    p.K = static_cast<int>(a.K);
    p.pad = a.group > 0 && !geom::is_unpadded(a.K, a.group);
    p.group = static_cast<int>(a.group > 0 ? a.group : a.K);
    p.stride = static_cast<int>(geom::group_stride(p.group));
    p.G = static_cast<int>(geom::num_groups(a.K, p.group));
    const int nvec = static_cast<int>(a.K / 8);
    const dim3 grid(static_cast<unsigned>(a.M));
    const bool res = a.residual != nullptr;
#define W4A8_RMS(V, NT)                                                                                  \
    {                                                                                                    \
        if (res) rmsnorm_quant_kernel<V, NT, true><<<grid, dim3(NT), 0, stream>>>(p);                    \
        else rmsnorm_quant_kernel<V, NT, false><<<grid, dim3(NT), 0, stream>>>(p);                       \
    }
    // A few rows (decode) are latency bound: one 8-element unit per thread
    // shortens each thread's serial work between the two block reductions.
    // Many rows fill the GPU either way and keep 256-thread workgroups.
    const bool few = a.M <= 64;
    if (nvec <= 256) W4A8_RMS(1, 256)
    else if (few && nvec <= 512) W4A8_RMS(1, 512)
    else if (few && nvec <= 1024) W4A8_RMS(1, 1024)
    else if (nvec <= 512) W4A8_RMS(2, 256)
    else if (nvec <= 1024) W4A8_RMS(4, 256)
    else if (nvec <= 2048) W4A8_RMS(2, 1024)
    else if (nvec <= 4096) W4A8_RMS(4, 1024)
    else if (nvec <= 8192) W4A8_RMS(8, 1024)
    else return hipErrorInvalidValue;
#undef W4A8_RMS
    return hipGetLastError();
}

}  // namespace w4a8
