// Decode-shaped W4A8 GEMM (M <= 64): HBM weight-stream bound.
//
// Computes, for symmetric int4 weights and per-token activation scales,
//   P_g[m,n] = sum_{k in g} a_q[m,k] * w[n,k]                       (int32, exact)
//   y[m,n]   = bf16( a_scale[m] * sum_g P_g[m,n] * w_scale[g,n] )    (fp32)
// the reference's grouped GEMM (npu_ops/kernel/midgroup_w4a8_gemm.inc:491-1169;
// CPU definition fakequant_lab/fake_linear.py:155-179) in its per-token,
// symmetric special case.
//
// Work split.  A workgroup owns CPW column blocks of 16 (16*CPW output
// columns) and ALL of K; its KW waves split K into contiguous, group-aligned
// ranges.  Each wave streams its range: per 128-K tile one 16-byte load per
// lane per column block (the repacked tile, 1 KB) plus MT*2 16-byte loads of
// activations (L2-resident; rows >= M are masked), held D tiles ahead in a
// register ring.  Every load is unconditional -- addresses are clamped into
// the buffers and the values masked afterwards -- so the compiler can count
// loads in flight exactly and the ring really overlaps.  Per 64-K slab each
// wave issues MT*CPW v_mfma_i32_16x16x64_i8; at each group end the int32
// accumulators fold into fp32 (acc += float(16*P) * w_scale).  The KW partial
// sums are reduced through LDS in a fixed order, and the token scale and the
// 1/16 of the nibble unpack are applied once at the end.  No workspace, no
// inter-workgroup communication, deterministic results.
#include <algorithm>

#include "common.h"
#include "kgeom.h"
#include "launch.h"

namespace w4a8 {
namespace {

struct DecodeParams {
    const int8_t* A;
    int64_t lda;
    const uint16_t* a_scale;
    const uint4* W;
    const uint16_t* S;
    uint16_t* Y;
    int64_t ldy;
    int32_t* P;        // optional partial dump [NG, M, N]
    int M, N, K;
    int KT, NG, NB;
    int spg;           // 64-K slabs per group
    int unit;          // tiles per K-split unit (group and tile aligned)
    int units;         // ceil(KT / unit)
};

template <int MT, int CPW, int KW, int D, bool SBF16, bool DUMP>
__global__ __launch_bounds__(64 * KW) void gemm_decode_kernel(const DecodeParams p) {
    constexpr int R = 16 * MT;
    constexpr int C = 16 * CPW;
    __shared__ float red[KW * R * C];

    const int lane = threadIdx.x & 63;
    // Wave-uniform by construction; readfirstlane tells the compiler so, which
    // keeps the tile loop and fold conditions scalar branches.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb0 = blockIdx.x * CPW;
    const int rowq = 4 * (lane >> 4);  // first output row of this lane in a 16-row tile
    const int colq = lane & 15;        // A row / output column of this lane in a 16-block

    // This wave's tile range [ta, tb).
    const int ua = (wave * p.units) / KW;
    const int ub = ((wave + 1) * p.units) / KW;
    const int ta = ua * p.unit;
    const int tb = min(p.KT, ub * p.unit);

    const uint4* wp[CPW];
    const uint16_t* sp[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const int nb = min(nb0 + c, p.NB - 1);
        wp[c] = p.W + static_cast<int64_t>(nb) * p.KT * 64 + lane;
        sp[c] = p.S + static_cast<int64_t>(nb) * p.NG * 16 + colq;
    }
    const int8_t* ap[MT];
    bool arow_ok[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int row = mt * 16 + colq;
        arow_ok[mt] = row < p.M;
        ap[mt] = p.A + static_cast<int64_t>(min(row, p.M - 1)) * p.lda + (lane >> 4) * 16;
    }

    uint4 wb[D][CPW];
    uint4 ab[D][MT][2];
    uint32_t sb[D][CPW][2];
    auto load_slot = [&](int s, int t) {
        const int tc = max(ta, min(t, tb - 1));   // clamp into this wave's range
#pragma unroll
        for (int c = 0; c < CPW; ++c) wb[s][c] = wp[c][static_cast<int64_t>(tc) * 64];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int h = 0; h < 2; ++h)   // a slab past K has zero weights; clamp its read into the row
                ab[s][mt][h] = *reinterpret_cast<const uint4*>(ap[mt] + min(tc * 128 + h * 64, p.K - 64));
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int g = min((2 * tc + h) / p.spg, p.NG - 1);
#pragma unroll
            for (int c = 0; c < CPW; ++c) sb[s][c][h] = sp[c][g * 16];
        }
    };

    float acc[MT][CPW][4];
    v4i P[MT][CPW];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
            P[mt][c] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[mt][c][i] = 0.0f;
        }

    if (tb > ta) {
#pragma unroll
        for (int s = 0; s < D; ++s) load_slot(s, ta + s);
        const int iters = (tb - ta + D - 1) / D;
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int s = 0; s < D; ++s) {
                const int t = ta + it * D + s;
                const bool tvalid = t < tb;
                uint4 wc[CPW];
                v4i a[MT][2];
                uint32_t sc[CPW][2];
#pragma unroll
                for (int c = 0; c < CPW; ++c) {
                    wc[c] = wb[s][c];
                    sc[c][0] = sb[s][c][0];
                    sc[c][1] = sb[s][c][1];
                }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint4 v = ab[s][mt][h];
                        const bool ok = arow_ok[mt];
                        a[mt][h] = v4i{ok ? static_cast<int>(v.x) : 0, ok ? static_cast<int>(v.y) : 0,
                                       ok ? static_cast<int>(v.z) : 0, ok ? static_cast<int>(v.w) : 0};
                    }
                load_slot(s, t + D);
                v4i b[CPW][2];
#pragma unroll
                for (int c = 0; c < CPW; ++c) {
                    unpack_tile_lane(wc[c], b[c][0], b[c][1]);
                    if (!tvalid) b[c][0] = b[c][1] = v4i{0, 0, 0, 0};
                }
#pragma unroll
                for (int h = 0; h < 2; ++h) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int c = 0; c < CPW; ++c) P[mt][c] = mfma16(a[mt][h], b[c][h], P[mt][c]);
                    const int sg = 2 * t + h;
                    const int g = sg / p.spg;
                    if (tvalid && ((sg + 1) % p.spg) == 0 && g < p.NG) {
#pragma unroll
                        for (int c = 0; c < CPW; ++c) {
                            const float ws = scale_to_f32<SBF16>(sc[c][h]);
#pragma unroll
                            for (int mt = 0; mt < MT; ++mt) {
                                if constexpr (DUMP) {
                                    const int col = (nb0 + c) * 16 + colq;
#pragma unroll
                                    for (int i = 0; i < 4; ++i) {
                                        const int row = mt * 16 + rowq + i;
                                        if (row < p.M && col < p.N)
                                            p.P[(static_cast<int64_t>(g) * p.M + row) * p.N + col] = P[mt][c][i] >> 4;
                                    }
                                }
#pragma unroll
                                for (int i = 0; i < 4; ++i) acc[mt][c][i] += static_cast<float>(P[mt][c][i]) * ws;
                                P[mt][c] = v4i{0, 0, 0, 0};
                            }
                        }
                    }
                }
            }
        }
    }

    // Fixed-order reduction of the KW wave partials, then the epilogue.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int c = 0; c < CPW; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave * R * C + (mt * 16 + rowq + i) * C + c * 16 + colq] = acc[mt][c][i];
    __syncthreads();
    for (int e = threadIdx.x; e < R * C; e += 64 * KW) {
        const int row = e / C;
        const int col = nb0 * 16 + (e - row * C);
        if (row >= p.M || col >= p.N) continue;
        float sum = red[e];
#pragma unroll
        for (int w = 1; w < KW; ++w) sum += red[w * R * C + e];
        const float ts = bf16_bits_to_f32(p.a_scale[row]) * 0.0625f;
        p.Y[static_cast<int64_t>(row) * p.ldy + col] = static_cast<uint16_t>(f32_to_bf16_bits(sum * ts));
    }
}

int gcd_i(int a, int b) {
    while (b) {
        const int t = a % b;
        a = b;
        b = t;
    }
    return a;
}

template <int MT, int CPW, int KW, int D, bool SBF16, bool DUMP>
hipError_t launch_cfg(const DecodeParams& p, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((p.NB + CPW - 1) / CPW));
    gemm_decode_kernel<MT, CPW, KW, D, SBF16, DUMP><<<grid, dim3(64 * KW), 0, stream>>>(p);
    return hipGetLastError();
}

template <bool SBF16, bool DUMP>
hipError_t launch_sd(const DecodeParams& p, hipStream_t stream) {
    const int mt = (p.M + 15) / 16;
    switch (mt) {
        case 1: return launch_cfg<1, 1, 8, 8, SBF16, DUMP>(p, stream);
        case 2: return launch_cfg<2, 2, 4, 4, SBF16, DUMP>(p, stream);
        case 3: return launch_cfg<3, 2, 4, 4, SBF16, DUMP>(p, stream);
        default: return launch_cfg<4, 2, 4, 4, SBF16, DUMP>(p, stream);
    }
}

}  // namespace

int64_t decode_workspace_bytes(int64_t, int64_t, int64_t, int64_t) { return 0; }

hipError_t launch_gemm_decode(const GemmArgs& a, hipStream_t stream) {
    DecodeParams p{};
    p.A = a.a_q;
    p.lda = a.lda;
    p.a_scale = a.a_scale;
    p.W = reinterpret_cast<const uint4*>(a.w_tiles);
    p.S = a.s_tiles;
    p.Y = a.y;
    p.ldy = a.ldy;
    p.P = a.partials;
    p.M = static_cast<int>(a.M);
    p.N = static_cast<int>(a.N);
    p.K = static_cast<int>(a.K);
    p.KT = static_cast<int>(geom::k_tiles(a.K, a.group));
    p.NG = static_cast<int>(geom::num_groups(a.K, a.group));
    p.NB = static_cast<int>(geom::col_blocks(a.N));
    p.spg = static_cast<int>(a.group / 64);
    // K-split boundaries fall on both tile (2 slabs) and group boundaries.
    p.unit = (2 * p.spg / gcd_i(2, p.spg)) / 2;
    p.units = (p.KT + p.unit - 1) / p.unit;
    const bool dump = a.partials != nullptr;
    if (a.scale_bf16) return dump ? launch_sd<true, true>(p, stream) : launch_sd<true, false>(p, stream);
    return dump ? launch_sd<false, true>(p, stream) : launch_sd<false, false>(p, stream);
}

}  // namespace w4a8
