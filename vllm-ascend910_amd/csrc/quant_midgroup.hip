// Mid-group activation quant in the reference's compat format (gfx950).
//
// The reference's `midgroup_quant_a` (kernel npu_ops/kernel/midgroup_quant_a.inc,
// host npu_ops/host/midgroup_quant_a.cpp:40-78): per (token, K-group) int8
// quant of a bf16 activation, emitted as the four tensors its mid-group GEMM
// reads, in the padded layouts of npu_ops/kernel/mg_kgeom.h:
//   a_hi    int8  [Mp, kpad/2]  packed int4 (even k in the low nibble), hi = q >> 4
//   a_lo    int8  [Mp, kpad/2]  packed int4, lo = (q & 15) - 8, i.e. nibble (q & 15) ^ 8
//   a_scale bf16  [G, Mp]       per (group, row)
//   a_ksum  int32 [G, Mp]       -sum_{k in g} q
// so that q = 16*hi + lo + 8.  Semantics per group are fakequant_lab/quant.py
// (group_params, :89-105, and quantize_with, :135-141): s = bf16_rne(max|x| / 127)
// with an IEEE divide, bf16 tiny when that is zero, q = clamp(rint(x / s)).
// Padding slots of a short last group hold q = 0 (hi nibble 0, lo nibble 8, the
// packer's 0x88), and rows [M, Mp) are written as scale tiny, q = 0, ksum 0,
// as the reference kernel does (midgroup_quant_a.inc:14-28).
//
// One 128-thread workgroup per (row, group), or per (4 rows, group) for large
// calls, handles up to 1024 padded slots of each row, 8 per thread (one
// 16-byte load where aligned, the rows' loads in flight together and kept in
// registers from the absmax to the quant); larger groups loop and read their
// later slots twice.  A two-pass form with 2-byte loads and an IEEE divide
// per element took 261 us at 4096 x 27648 (this one 85).
// The quotient rint(x / s) is taken in the reciprocal form of common.h
// (row_scale / quant_code), equal to the IEEE divide for these scales.
#include "common.h"
#include "kgeom.h"
#include "launch.h"

namespace w4a8 {
namespace {

constexpr int kThreadsMG = 128;
constexpr uint32_t kTinyBits = 0x0080u;   // bf16 2^-126, torch.finfo(torch.bfloat16).tiny

struct MidQuantParams {
    const uint16_t* x;
    int64_t ldx;
    uint8_t* a_hi;
    uint8_t* a_lo;
    uint16_t* a_scale;
    int32_t* a_ksum;
    int64_t lda;       // plane row pitch in bytes (kpad / 2)
    int M, Mp, K;
    int group, stride, G;
};

// Eight consecutive bf16 of the group (as four packed dwords), zero past the
// group's real members: one 16-byte load where the slots are whole and the
// address 16-byte aligned (`vec`, uniform per workgroup), element loads
// otherwise.
__device__ __forceinline__ uint4 load8(const uint16_t* xr, int k0, int real, bool vec) {
    if (vec && k0 + 8 <= real) return *reinterpret_cast<const uint4*>(xr + k0);
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = k0 + 2 * j;
        const uint32_t lo = k < real ? xr[k] : 0u;
        const uint32_t hi = k + 1 < real ? xr[k + 1] : 0u;
        w[j] = lo | (hi << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// Eight codes -> four bytes of each plane (slot j in nibble j: even k low).
template <bool FAST>
__device__ __forceinline__ void pack8(const uint4& v, const RowScale& q, uint32_t& hw, uint32_t& lw, int& ksum) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    hw = 0u;
    lw = 0u;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t u = w[j >> 1];
        const int c = quant_code<FAST>(__uint_as_float((j & 1) ? (u & 0xffff0000u) : (u << 16)), q);
        ksum += c;
        hw |= (static_cast<uint32_t>(c >> 4) & 0xfu) << (4 * j);
        lw |= ((static_cast<uint32_t>(c) & 0xfu) ^ 0x8u) << (4 * j);
    }
}

// kRowsMG rows per workgroup, their first loads all in flight together.
template <int kRowsMG>
__global__ __launch_bounds__(kThreadsMG) void quant_midgroup_kernel(const MidQuantParams p) {
    __shared__ uint32_t red_max[kRowsMG][kThreadsMG / 64];
    __shared__ int red_sum[kRowsMG][kThreadsMG / 64];
    const int row0 = blockIdx.x * kRowsMG;
    const int g = blockIdx.y;
    const int tid = threadIdx.x;
    const int real = (g + 1 < p.G) ? p.group : p.K - (p.G - 1) * p.group;
    const int padded = static_cast<int>(geom::ceil_to(real, geom::kGroupAlign));
    const int chunks = padded / 8;   // 8-slot chunks (padded is a multiple of 64)
    auto src = [&](int r) {
        return p.x + static_cast<int64_t>(row0 + r) * p.ldx + static_cast<int64_t>(g) * p.group;
    };
    // 16-byte loads where every row's group start is 16-byte aligned (uniform)
    const bool vec = ((reinterpret_cast<uintptr_t>(src(0)) | static_cast<uintptr_t>(p.ldx * 2)) & 15u) == 0;

    // pass 1: max |x| over each row's real members (bf16 magnitude order =
    // order of the 15 low bits for finite values); every row's first chunk of
    // this thread is requested before any is used, and stays in registers for
    // pass 2 (all of a group of up to 1024)
    uint4 v0[kRowsMG];
    uint32_t amax[kRowsMG];
#pragma unroll
    for (int r = 0; r < kRowsMG; ++r) {
        const bool live = row0 + r < p.M;
        v0[r] = (live && tid < chunks) ? load8(src(r), 8 * tid, real, vec) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int r = 0; r < kRowsMG; ++r) {
        amax[r] = abs_bits_max8(v0[r]);
        if (row0 + r < p.M)
            for (int c = tid + kThreadsMG; c < chunks; c += kThreadsMG) amax[r] = max(amax[r], abs_bits_max8(load8(src(r), 8 * c, real, vec)));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1)
            amax[r] = max(amax[r], static_cast<uint32_t>(__shfl_xor(static_cast<int>(amax[r]), off, 64)));
        if ((tid & 63) == 0) red_max[r][tid >> 6] = amax[r];
    }
    __syncthreads();

    // pass 2: 8 padded slots per thread and trip -> 4 bytes of each plane
    int ksum[kRowsMG];
    uint32_t sbits[kRowsMG];
#pragma unroll
    for (int r = 0; r < kRowsMG; ++r) {
        const int row = row0 + r;
        ksum[r] = 0;
        const uint32_t am = max(red_max[r][0], red_max[r][1]);
        sbits[r] = f32_to_bf16_bits(bf16_bits_to_f32(am) / 127.0f);
        if ((sbits[r] & 0x7fffu) == 0u) sbits[r] = kTinyBits;
        if (row >= p.Mp) continue;
        // q = clamp(rint(x / s)): the reciprocal form with its tie correction
        // (common.h: exact for these scales, |x| <= 127.25 s), else a divide
        const RowScale q = row_scale(bf16_bits_to_f32(sbits[r]));
        const bool live = row < p.M;
        uint8_t* hrow = p.a_hi + static_cast<int64_t>(row) * p.lda + static_cast<int64_t>(g) * (p.stride / 2);
        uint8_t* lrow = p.a_lo + static_cast<int64_t>(row) * p.lda + static_cast<int64_t>(g) * (p.stride / 2);
        for (int c = tid; c < chunks; c += kThreadsMG) {
            const uint4 v = c == tid ? v0[r] : (live ? load8(src(r), 8 * c, real, vec) : make_uint4(0u, 0u, 0u, 0u));
            uint32_t hw, lw;
            if (q.fast) pack8<true>(v, q, hw, lw, ksum[r]);
            else pack8<false>(v, q, hw, lw, ksum[r]);
            *reinterpret_cast<uint32_t*>(hrow + 4 * c) = hw;
            *reinterpret_cast<uint32_t*>(lrow + 4 * c) = lw;
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ksum[r] += __shfl_xor(ksum[r], off, 64);
        if ((tid & 63) == 0) red_sum[r][tid >> 6] = ksum[r];
    }
    __syncthreads();
    if (tid < kRowsMG && row0 + tid < p.Mp) {
        const int r = tid;
        uint32_t sb = 0u;
#pragma unroll
        for (int i = 0; i < kRowsMG; ++i)
            if (i == r) sb = sbits[i];
        p.a_scale[static_cast<int64_t>(g) * p.Mp + row0 + r] = static_cast<uint16_t>(sb);
        p.a_ksum[static_cast<int64_t>(g) * p.Mp + row0 + r] = -(red_sum[r][0] + red_sum[r][1]);
    }
}

}  // namespace

hipError_t launch_quant_midgroup(const uint16_t* x, int64_t ldx, uint8_t* a_hi, uint8_t* a_lo,
                                 uint16_t* a_scale, int32_t* a_ksum, int64_t M, int64_t Mp, int64_t K,
                                 int64_t group, hipStream_t stream) {
    if (Mp == 0) return hipSuccess;
    MidQuantParams p{};
    p.x = x;
    p.ldx = ldx;
    p.a_hi = a_hi;
    p.a_lo = a_lo;
    p.a_scale = a_scale;
    p.a_ksum = a_ksum;
    p.lda = geom::kpad(K, group) / 2;
    p.M = static_cast<int>(M);
    p.Mp = static_cast<int>(Mp);
    p.K = static_cast<int>(K);
    p.group = static_cast<int>(group);
    p.stride = static_cast<int>(geom::group_stride(group));
    p.G = static_cast<int>(geom::num_groups(K, group));
    // Rows per workgroup: one while the (row, group) workgroups are few, four
    // past 64k of them, where each one's single 2 KB round trip bounds the
    // call (MI355X, graph replays, group 1024, us, one row / four rows: 1 x
    // 5120 4.2 / 6.4, 4096 x 5120 19.6 / 22.2, 1024 x 27648 25.7 / 27.1,
    // 4096 x 27648 100.8 / 85.3; all the same bytes).
    if (Mp * p.G > 65536) {
        const dim3 grid(static_cast<unsigned>((Mp + 3) / 4), static_cast<unsigned>(p.G));
        quant_midgroup_kernel<4><<<grid, dim3(kThreadsMG), 0, stream>>>(p);
    } else {
        const dim3 grid(static_cast<unsigned>(Mp), static_cast<unsigned>(p.G));
        quant_midgroup_kernel<1><<<grid, dim3(kThreadsMG), 0, stream>>>(p);
    }
    return hipGetLastError();
}

}  // namespace w4a8
