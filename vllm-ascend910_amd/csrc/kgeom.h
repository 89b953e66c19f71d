// Group geometry along K for the W4A8 per-group linear.
//
// Follows the reference's ragged-K contract (npu_ops/kernel/mg_kgeom.h:47-129):
// G = ceil(K / group) quant groups, only the last one may be short, and in the
// PACKED weight layout every group starts at g * ceil_to(group, 64) and is
// zero-padded up to a multiple of 64 elements.  A zero-padded slot holds the
// int4 code 0, so it adds nothing to any integer dot product; that is why
// sums may be taken over the padded span.
//
// Shared by the HIP kernels, the C-ABI host checks and the repacker.  Plain
// constexpr arithmetic, usable from host and device code.
#pragma once

#include <stdint.h>

namespace w4a8 {
namespace geom {

// The reference's packed-layout alignment: 64 int4 elements per group step.
constexpr int64_t kGroupAlign = 64;
// One MFMA K-slab (v_mfma_i32_16x16x64_i8 consumes 64 K per instruction).
constexpr int64_t kSlabK = 64;
// One repacked weight tile covers 16 output columns x 128 K = 1024 bytes.
constexpr int64_t kTileN = 16;
constexpr int64_t kTileK = 128;
constexpr int64_t kTileBytes = kTileN * kTileK / 2;

__host__ __device__ constexpr int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ constexpr int64_t ceil_to(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// Number of quant groups along K; the last one may be short.
__host__ __device__ constexpr int64_t num_groups(int64_t K, int64_t group) { return ceil_div(K, group); }

// Padded width of a full group, which is also the offset step between groups.
__host__ __device__ constexpr int64_t group_stride(int64_t group) { return ceil_to(group, kGroupAlign); }

// Real (unpadded) element count of group g.
__host__ __device__ constexpr int64_t group_real(int64_t g, int64_t K, int64_t group) {
    return (g + 1 < num_groups(K, group)) ? group : K - (num_groups(K, group) - 1) * group;
}

// Padded element count of group g.
__host__ __device__ constexpr int64_t group_pad(int64_t g, int64_t K, int64_t group) {
    return ceil_to(group_real(g, K, group), kGroupAlign);
}

// Element offset of group g inside a padded row.
__host__ __device__ constexpr int64_t group_offset(int64_t g, int64_t group) { return g * group_stride(group); }

// Padded row length in elements (the packed weight row is kpad/2 bytes).
__host__ __device__ constexpr int64_t kpad(int64_t K, int64_t group) {
    return (num_groups(K, group) - 1) * group_stride(group) +
           group_pad(num_groups(K, group) - 1, K, group);
}

// Repacked layout sizes: NB column blocks of 16, KT tiles of 128 padded-K.
__host__ __device__ constexpr int64_t col_blocks(int64_t N) { return ceil_div(N, kTileN); }
__host__ __device__ constexpr int64_t k_tiles(int64_t K, int64_t group) { return ceil_div(kpad(K, group), kTileK); }

// True when the padded layout is the plain one (kpad == K): every group a
// whole number of 64-element slabs, e.g. K % group == 0 and group % 64 == 0.
__host__ __device__ constexpr bool is_unpadded(int64_t K, int64_t group) {
    return group > 0 && K > 0 && kpad(K, group) == K;
}

}  // namespace geom
}  // namespace w4a8
