// Offline repacker: reference packed-int4 weight -> gfx950 MFMA operand order.
//
// Input (reference layout, npu_ops/python/w4a8_ops.py:142-148 and :231-239):
//   w_q [N, kpad/2] bytes, two int4 codes per byte along K, even k in the low
//   nibble, group g at padded offset g*ceil_to(group,64).
//
// Output: tiles of 16 columns x 128 padded-K, 1024 bytes each, ordered
// [col block nb][k tile kt].  Inside a tile, lane l (0..63) owns 16 bytes at
// offset 16*l: column nb*16 + l%16 and, for slab h in {0,1}, the 16 codes
//   k = kt*128 + h*64 + (l/16)*16 + [0, 16)
// which is exactly what lane l feeds to v_mfma_i32_16x16x64_i8 as its B
// operand for that slab (B lane l = column l%16, K chunk l/16).  Dword d of
// the 16 bytes covers 8 codes k0 = kt*128 + (d/2)*64 + (l/16)*16 + (d%2)*8;
// its byte j holds code k0+j in the low nibble and code k0+4+j in the high
// nibble, so two AND/shift operations produce two int8x4 words in natural K
// order (see unpack_lo4/unpack_hi4).  Columns >= N and K >= kpad are zero.
//
// Scales are regrouped from [G, N] to [nb][G][16] so that a wave streaming one
// column block reads its scales contiguously.
#include "common.h"
#include "kgeom.h"
#include "launch.h"

namespace w4a8 {
namespace {

__global__ __launch_bounds__(256) void repack_weight_kernel(const uint8_t* __restrict__ wq,
                                                             uint32_t* __restrict__ out,
                                                             int64_t N, int64_t kpadv,
                                                             int64_t KT, int64_t total_dwords) {
    const int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (o >= total_dwords) return;
    const int64_t tile = o >> 8;
    const int lane = static_cast<int>((o >> 2) & 63);
    const int d = static_cast<int>(o & 3);
    const int64_t nb = tile / KT;
    const int64_t kt = tile - nb * KT;
    const int64_t n = nb * 16 + (lane & 15);
    const int64_t k0 = kt * 128 + (d >> 1) * 64 + (lane >> 4) * 16 + (d & 1) * 8;
    uint32_t in = 0u;
    if (n < N && k0 < kpadv) {
        in = *reinterpret_cast<const uint32_t*>(wq + n * (kpadv / 2) + k0 / 2);
    }
    // in nibble i = code k0+i; out nibble 2j = code k0+j, out nibble 2j+1 = code k0+4+j.
    uint32_t r = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        r |= ((in >> (4 * j)) & 0xfu) << (8 * j);
        r |= ((in >> (4 * (j + 4))) & 0xfu) << (8 * j + 4);
    }
    out[o] = r;
}

__global__ __launch_bounds__(256) void repack_scale_kernel(const uint16_t* __restrict__ ws,
                                                            uint16_t* __restrict__ out,
                                                            int64_t N, int64_t G,
                                                            int64_t total) {
    const int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (o >= total) return;
    const int64_t i = o & 15;
    const int64_t g = (o >> 4) % G;
    const int64_t nb = (o >> 4) / G;
    const int64_t n = nb * 16 + i;
    out[o] = (n < N) ? ws[g * N + n] : static_cast<uint16_t>(0);
}

}  // namespace

hipError_t launch_repack_weights(const uint8_t* w_q, uint8_t* w_tiles, int64_t N, int64_t K, int64_t group,
                                 hipStream_t stream) {
    const int64_t kp = geom::kpad(K, group);
    const int64_t KT = geom::k_tiles(K, group);
    const int64_t wd = geom::col_blocks(N) * KT * 256;  // dwords
    if (wd > 0)
        repack_weight_kernel<<<dim3(static_cast<unsigned>((wd + 255) / 256)), dim3(256), 0, stream>>>(
            w_q, reinterpret_cast<uint32_t*>(w_tiles), N, kp, KT, wd);
    return hipGetLastError();
}

hipError_t launch_repack(const uint8_t* w_q, const uint16_t* w_scale, uint8_t* w_tiles,
                         uint16_t* s_tiles, int64_t N, int64_t K, int64_t group,
                         hipStream_t stream) {
    const int64_t kp = geom::kpad(K, group);
    const int64_t NB = geom::col_blocks(N);
    const int64_t KT = geom::k_tiles(K, group);
    const int64_t G = geom::num_groups(K, group);
    const int64_t wd = NB * KT * 256;  // dwords
    if (wd > 0) {
        const int64_t blocks = (wd + 255) / 256;
        repack_weight_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(
            w_q, reinterpret_cast<uint32_t*>(w_tiles), N, kp, KT, wd);
    }
    const int64_t sn = NB * G * 16;
    if (sn > 0) {
        const int64_t blocks = (sn + 255) / 256;
        repack_scale_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(
            w_scale, s_tiles, N, G, sn);
    }
    return hipGetLastError();
}

}  // namespace w4a8
