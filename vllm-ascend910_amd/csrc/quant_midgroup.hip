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
// One 128-thread workgroup per (row, group) handles up to 1024 padded slots,
// 8 per thread; larger groups loop.
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

__device__ __forceinline__ int quant_one(uint32_t xbits, float s) {
    float q = rintf(bf16_bits_to_f32(xbits) / s);
    q = fminf(127.0f, fmaxf(-128.0f, q));
    return static_cast<int>(q);
}

__global__ __launch_bounds__(kThreadsMG) void quant_midgroup_kernel(const MidQuantParams p) {
    __shared__ uint32_t red_max[kThreadsMG / 64];
    __shared__ int red_sum[kThreadsMG / 64];
    const int row = blockIdx.x;
    const int g = blockIdx.y;
    const int tid = threadIdx.x;
    const int real = (g + 1 < p.G) ? p.group : p.K - (p.G - 1) * p.group;
    const int padded = static_cast<int>(geom::ceil_to(real, geom::kGroupAlign));
    const bool live = row < p.M;
    const uint16_t* xr = p.x + static_cast<int64_t>(row) * p.ldx + static_cast<int64_t>(g) * p.group;

    // pass 1: max |x| over the group's real members (bf16 magnitude order =
    // order of the 15 low bits for finite values)
    uint32_t amax = 0u;
    if (live)
        for (int k = tid; k < real; k += kThreadsMG) amax = max(amax, static_cast<uint32_t>(xr[k]) & 0x7fffu);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) amax = max(amax, static_cast<uint32_t>(__shfl_xor(static_cast<int>(amax), off, 64)));
    if ((tid & 63) == 0) red_max[tid >> 6] = amax;
    __syncthreads();
    amax = max(red_max[0], red_max[1]);
    uint32_t sbits = f32_to_bf16_bits(bf16_bits_to_f32(amax) / 127.0f);
    if ((sbits & 0x7fffu) == 0u) sbits = kTinyBits;
    const float s = bf16_bits_to_f32(sbits);

    // pass 2: 8 padded slots per thread -> 4 bytes of each plane
    int ksum = 0;
    uint8_t* hrow = p.a_hi + static_cast<int64_t>(row) * p.lda + static_cast<int64_t>(g) * (p.stride / 2);
    uint8_t* lrow = p.a_lo + static_cast<int64_t>(row) * p.lda + static_cast<int64_t>(g) * (p.stride / 2);
    for (int k0 = tid * 8; k0 < padded; k0 += kThreadsMG * 8) {
        uint32_t hw = 0u, lw = 0u;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int k = k0 + j;
            const int q = (live && k < real) ? quant_one(xr[k], s) : 0;
            ksum += q;
            hw |= (static_cast<uint32_t>(q >> 4) & 0xfu) << (4 * j);
            lw |= ((static_cast<uint32_t>(q) & 0xfu) ^ 0x8u) << (4 * j);
        }
        *reinterpret_cast<uint32_t*>(hrow + k0 / 2) = hw;
        *reinterpret_cast<uint32_t*>(lrow + k0 / 2) = lw;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ksum += __shfl_xor(ksum, off, 64);
    if ((tid & 63) == 0) red_sum[tid >> 6] = ksum;
    __syncthreads();
    if (tid == 0) {
        p.a_scale[static_cast<int64_t>(g) * p.Mp + row] = static_cast<uint16_t>(sbits);
        p.a_ksum[static_cast<int64_t>(g) * p.Mp + row] = -(red_sum[0] + red_sum[1]);
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
    const dim3 grid(static_cast<unsigned>(Mp), static_cast<unsigned>(p.G));
    quant_midgroup_kernel<<<grid, dim3(kThreadsMG), 0, stream>>>(p);
    return hipGetLastError();
}

}  // namespace w4a8
