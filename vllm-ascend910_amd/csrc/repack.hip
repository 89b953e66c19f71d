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

// One output nibble order per input dword: in nibble i = code k0+i; out
// nibble 2j = code k0+j, out nibble 2j+1 = code k0+4+j.
__device__ __forceinline__ uint32_t tile_dword(uint32_t in) {
    uint32_t r = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        r |= ((in >> (4 * j)) & 0xfu) << (8 * j);
        r |= ((in >> (4 * (j + 4))) & 0xfu) << (8 * j + 4);
    }
    return r;
}

// One thread per 16-byte lane chunk of a tile: its dwords d = 0, 1 are the
// 8 bytes at K byte kt*64 + (l/16)*8 of column n's row, d = 2, 3 the 8 bytes
// 32 further (16 codes each, inside or past kpad as a whole).
__global__ __launch_bounds__(256) void repack_weight_kernel(const uint8_t* __restrict__ wq,
                                                             uint4* __restrict__ out,
                                                             int64_t N, int64_t kpadv,
                                                             int64_t KT, int64_t total_chunks) {
    const int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (o >= total_chunks) return;
    const int64_t tile = o >> 6;
    const int lane = static_cast<int>(o & 63);
    const int64_t nb = tile / KT;
    const int64_t kt = tile - nb * KT;
    const int64_t n = nb * 16 + (lane & 15);
    uint32_t in[4] = {0u, 0u, 0u, 0u};
    if (n < N) {
        const uint8_t* row = wq + n * (kpadv / 2);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t b = kt * 64 + h * 32 + (lane >> 4) * 8;
            if (2 * b < kpadv) {   // dword loads: w_q is only required 4-byte aligned
                in[2 * h] = *reinterpret_cast<const uint32_t*>(row + b);
                in[2 * h + 1] = *reinterpret_cast<const uint32_t*>(row + b + 4);
            }
        }
    }
    out[o] = make_uint4(tile_dword(in[0]), tile_dword(in[1]), tile_dword(in[2]), tile_dword(in[3]));
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
    const int64_t wc = geom::col_blocks(N) * KT * 64;  // 16-byte lane chunks
    if (wc > 0)
        repack_weight_kernel<<<dim3(static_cast<unsigned>((wc + 255) / 256)), dim3(256), 0, stream>>>(
            w_q, reinterpret_cast<uint4*>(w_tiles), N, kp, KT, wc);
    return hipGetLastError();
}

hipError_t launch_repack(const uint8_t* w_q, const uint16_t* w_scale, uint8_t* w_tiles,
                         uint16_t* s_tiles, int64_t N, int64_t K, int64_t group,
                         hipStream_t stream) {
    const int64_t kp = geom::kpad(K, group);
    const int64_t NB = geom::col_blocks(N);
    const int64_t KT = geom::k_tiles(K, group);
    const int64_t G = geom::num_groups(K, group);
    const int64_t wc = NB * KT * 64;  // 16-byte lane chunks
    if (wc > 0) {
        const int64_t blocks = (wc + 255) / 256;
        repack_weight_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(
            w_q, reinterpret_cast<uint4*>(w_tiles), N, kp, KT, wc);
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
