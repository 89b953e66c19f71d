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
#include <type_traits>

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

template <int MT, int CPW, int KWMAX, int D, bool G64, bool SBF16, bool DUMP>
__global__ __launch_bounds__(64 * KWMAX) void gemm_decode_kernel(const DecodeParams p) {
    constexpr int R = 16 * MT;
    constexpr int C = 16 * CPW;
    // kw * R * C floats, sized at launch for the waves actually launched.
    extern __shared__ float red[];

    const int lane = threadIdx.x & 63;
    // Wave-uniform by construction; readfirstlane tells the compiler so, which
    // keeps the tile loop and fold conditions scalar branches.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kw = blockDim.x >> 6;
    const int nb0 = blockIdx.x * CPW;
    const int rowq = 4 * (lane >> 4);  // first output row of this lane in a 16-row tile
    const int colq = lane & 15;        // A row / output column of this lane in a 16-block

    // This wave's tile range [ta, tb).
    const int ua = (wave * p.units) / kw;
    const int ub = ((wave + 1) * p.units) / kw;
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

    // Register ring: D tiles of weights, activations and the scales of the
    // groups ending in them (two per tile for group 64, one otherwise: a group
    // of >= 128 can only end on a tile's upper slab).
    constexpr int NS = G64 ? 2 : 1;
    uint4 wb[D][CPW];
    uint4 ab[D][MT][2];
    uint32_t sb[D][CPW][NS];
    auto load_slot = [&](int s, int t) {
        const int tc = max(ta, min(t, tb - 1));   // clamp into this wave's range
#pragma unroll
        for (int c = 0; c < CPW; ++c) wb[s][c] = load_stream(wp[c] + static_cast<int64_t>(tc) * 64);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int h = 0; h < 2; ++h)   // a slab past K has zero weights; clamp its read into the row
                ab[s][mt][h] = *reinterpret_cast<const uint4*>(ap[mt] + min(tc * 128 + h * 64, p.K - 64));
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            const int g = min((2 * tc + (G64 ? j : 1)) / p.spg, p.NG - 1);
#pragma unroll
            for (int c = 0; c < CPW; ++c) sb[s][c][j] = sp[c][g * 16];
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

    // One pass over the D ring slots; PREFETCH refills each slot with the tile
    // D ahead (the last pass is peeled without it, so nothing past the range
    // is requested).
    auto pass = [&](int it, auto prefetch) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const int t = ta + it * D + s;
            const bool tvalid = t < tb;
            uint4 wc[CPW];
            v4i a[MT][2];
            uint32_t sc[CPW][NS];
#pragma unroll
            for (int c = 0; c < CPW; ++c) {
                wc[c] = wb[s][c];
#pragma unroll
                for (int j = 0; j < NS; ++j) sc[c][j] = sb[s][c][j];
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
            if constexpr (decltype(prefetch)::value) load_slot(s, t + D);
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
                if (!G64 && h == 0) continue;
                const int sg = 2 * t + h;
                const int g = sg / p.spg;
                if (tvalid && ((sg + 1) % p.spg) == 0 && g < p.NG) {
#pragma unroll
                    for (int c = 0; c < CPW; ++c) {
                        const float ws = scale_to_f32<SBF16>(sc[c][G64 ? h : 0]);
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
    };

    if (tb > ta) {
#pragma unroll
        for (int s = 0; s < D; ++s) load_slot(s, ta + s);
        const int iters = (tb - ta + D - 1) / D;
        for (int it = 0; it + 1 < iters; ++it) pass(it, std::true_type{});
        pass(iters - 1, std::false_type{});
    }

    // Fixed-order reduction of the kw wave partials, then the epilogue.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int c = 0; c < CPW; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave * R * C + (mt * 16 + rowq + i) * C + c * 16 + colq] = acc[mt][c][i];
    __syncthreads();
    for (int e = threadIdx.x; e < R * C; e += blockDim.x) {
        const int row = e / C;
        const int col = nb0 * 16 + (e - row * C);
        if (row >= p.M || col >= p.N) continue;
        float sum = red[e];
        for (int w = 1; w < kw; ++w) sum += red[w * R * C + e];
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

constexpr int kwmax_for(int mt) { return mt == 1 ? 16 : (mt == 2 ? 8 : 4); }

template <int MT, int CPW, int D, bool DUMP>
hipError_t launch_v(const DecodeParams& p, int kw, bool g64, bool sbf16, hipStream_t stream) {
    constexpr int KWM = kwmax_for(MT);
    const int w = std::max(1, std::min(kw, KWM));
    const dim3 grid(static_cast<unsigned>((p.NB + CPW - 1) / CPW)), block(64 * w);
    const size_t lds = static_cast<size_t>(w) * 16 * MT * 16 * CPW * sizeof(float);
    if (g64) {
        if (sbf16) gemm_decode_kernel<MT, CPW, KWM, D, true, true, DUMP><<<grid, block, lds, stream>>>(p);
        else gemm_decode_kernel<MT, CPW, KWM, D, true, false, DUMP><<<grid, block, lds, stream>>>(p);
    } else {
        if (sbf16) gemm_decode_kernel<MT, CPW, KWM, D, false, true, DUMP><<<grid, block, lds, stream>>>(p);
        else gemm_decode_kernel<MT, CPW, KWM, D, false, false, DUMP><<<grid, block, lds, stream>>>(p);
    }
    return hipGetLastError();
}

// The variants that are built: (MT, D, CPW).
template <bool DUMP>
hipError_t dispatch(const DecodeParams& p, const DecodeConfig& c, bool g64, bool sbf16, hipStream_t s) {
    const int mt = (p.M + 15) / 16;
    if (mt == 1 && c.D == 8 && c.CPW == 1) return launch_v<1, 1, 8, DUMP>(p, c.KW, g64, sbf16, s);
    if (mt == 1 && c.D == 4 && c.CPW == 1) return launch_v<1, 1, 4, DUMP>(p, c.KW, g64, sbf16, s);
    if (mt == 1 && c.D == 4 && c.CPW == 2) return launch_v<1, 2, 4, DUMP>(p, c.KW, g64, sbf16, s);
    if (mt == 2 && c.D == 4 && c.CPW == 1) return launch_v<2, 1, 4, DUMP>(p, c.KW, g64, sbf16, s);
    if (mt == 2 && c.D == 4 && c.CPW == 2) return launch_v<2, 2, 4, DUMP>(p, c.KW, g64, sbf16, s);
    if (mt == 3 && c.D == 4 && c.CPW == 2) return launch_v<3, 2, 4, DUMP>(p, c.KW, g64, sbf16, s);
    if (mt == 4 && c.D == 4 && c.CPW == 2) return launch_v<4, 2, 4, DUMP>(p, c.KW, g64, sbf16, s);
    if (mt == 4 && c.D == 2 && c.CPW == 4) return launch_v<4, 4, 2, DUMP>(p, c.KW, g64, sbf16, s);
    return hipErrorInvalidValue;
}

DecodeParams make_params(const GemmArgs& a) {
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
    return p;
}

}  // namespace

int64_t decode_workspace_bytes(int64_t, int64_t, int64_t, int64_t) { return 0; }

DecodeConfig decode_config(int64_t M, int64_t N, int64_t K, int64_t group) {
    // Picked from a sweep over ring depth, column blocks per workgroup and
    // waves per workgroup on MI355X at the QwQ-32B projection shapes.
    const int mt = static_cast<int>((M + 15) / 16);
    const int KT = static_cast<int>(geom::k_tiles(K, group));
    const int64_t NB = geom::col_blocks(N);
    DecodeConfig c{4, 2, 4};
    if (mt <= 2) {
        // Wide N already gives >= 1024 workgroups; otherwise split K so that
        // each wave holds about one ring (4 tiles) of its range.
        const int64_t wgs = (NB + 1) / 2;
        if (wgs >= 1024) c.KW = M <= 8 ? 2 : 1;
        else c.KW = std::max(1, std::min(mt == 1 ? 12 : 8, (KT + 3) / 4));
    } else if ((NB + 1) / 2 >= 1024) {
        c = DecodeConfig{2, 4, 1};
    }
    return c;
}

hipError_t launch_gemm_decode_cfg(const GemmArgs& a, const DecodeConfig& cfg, hipStream_t stream) {
    const DecodeParams p = make_params(a);
    const bool g64 = p.spg == 1;
    return a.partials ? dispatch<true>(p, cfg, g64, a.scale_bf16, stream)
                      : dispatch<false>(p, cfg, g64, a.scale_bf16, stream);
}

hipError_t launch_gemm_decode(const GemmArgs& a, hipStream_t stream) {
    return launch_gemm_decode_cfg(a, decode_config(a.M, a.N, a.K, a.group), stream);
}

}  // namespace w4a8
