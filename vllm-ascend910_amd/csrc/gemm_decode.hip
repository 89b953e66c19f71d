// Decode-shaped W4A8 GEMM (M <= 64): HBM weight-stream bound.
//
// Computes, for symmetric int4 weights and per-token activation scales,
//   P_g[m,n] = sum_{k in g} a_q[m,k] * w[n,k]                       (int32, exact)
//   y[m,n]   = bf16( a_scale[m] * sum_g P_g[m,n] * w_scale[g,n] )    (fp32)
// the reference's grouped GEMM (npu_ops/kernel/midgroup_w4a8_gemm.inc:491-1169;
// CPU definition fakequant_lab/fake_linear.py:155-179) in its per-token,
// symmetric special case.
//
// Work split.  Each 256-thread workgroup owns 4*CPW column blocks of 16 and a
// contiguous, group-aligned range of 128-K weight tiles (split-K over
// blockIdx.y).  Each wave streams its own column block(s): one 16-byte load
// per lane per tile (1 KB per wave), kept PF tiles ahead in a register ring so
// that many loads are in flight per CU.  The activations for the workgroup's
// K range are staged through LDS in chunks of TC tiles and shared by the four
// waves.  Per 64-K slab each wave issues MT*CPW v_mfma_i32_16x16x64_i8 (16 rows
// of A by 16 columns of B); at each group end the int32 accumulators are folded
// into fp32: acc += float(16*P) * w_scale.  The token scale and the 1/16 of the
// nibble unpack are applied once at the end (both exact power-of-two / single
// multiplies, see common.h).
//
// Split-K reduction is deterministic: every split writes its fp32 partial to
// the workspace, and the last workgroup to arrive at a column group (counted
// with a device-scope atomic) sums the partials in split order and writes bf16.
// It then resets the counter, so the workspace counters stay zero between calls.
#include <algorithm>

#include "common.h"
#include "kgeom.h"
#include "launch.h"

namespace w4a8 {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kPF = 8;             // tiles in flight per wave (register ring depth)
constexpr int kLdsBudget = 40960;  // bytes of A staging per workgroup
// Split-K arrival counters live in a FIXED region at the start of the
// workspace, one uint32 per column group, so that no call's partials ever
// overlap another call's counters: the region stays zero between calls.
constexpr int64_t kCounterBytes = 256 * 1024;
constexpr int64_t kMaxCounters = kCounterBytes / 4;

template <int MT>
struct DecodeCfg {
    static constexpr int kRows = 16 * MT;
    // Tiles per A chunk, so that rows * (TC*128 + 16) <= kLdsBudget.
    static constexpr int kTC = ((kLdsBudget / kRows) - 16) / 128;
    static constexpr int kLStride = kTC * 128 + 16;  // +16 B per row against bank conflicts
    static constexpr int kLdsBytes = kRows * kLStride;
};

struct DecodeParams {
    const int8_t* A;
    int64_t lda;
    const uint16_t* a_scale;
    const uint4* W;
    const uint16_t* S;
    uint16_t* Y;
    int64_t ldy;
    int32_t* P;        // optional partial dump [NG, M, N]
    float* part;       // split-K partials [ksplit, M, N]
    uint32_t* cnt;     // split-K arrival counters [ncg]
    int M, N, K;
    int KT, NG, NB;
    int spg;           // 64-K slabs per group
    int tps;           // tiles per split
    int ksplit;
};

template <int MT, int CPW, bool SBF16, bool DUMP>
__global__ __launch_bounds__(kThreads) void gemm_decode_kernel(const DecodeParams p) {
    using Cfg = DecodeCfg<MT>;
    __shared__ __attribute__((aligned(16))) int8_t lds[Cfg::kLdsBytes];
    __shared__ uint32_t s_last;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int t0 = blockIdx.y * p.tps;
    const int t1 = min(p.KT, t0 + p.tps);
    const int nbw = (blockIdx.x * kWaves + wave) * CPW;

    const uint4* wp[CPW];
    const uint16_t* sp[CPW];
    bool cval[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        cval[c] = (nbw + c) < p.NB;
        const int nb = cval[c] ? (nbw + c) : 0;
        wp[c] = p.W + static_cast<int64_t>(nb) * p.KT * 64 + lane;
        sp[c] = p.S + static_cast<int64_t>(nb) * p.NG * 16 + (lane & 15);
    }

    // Scale prefetch for the (at most two) groups that end inside tile t.
    auto load_scales = [&](int t, uint32_t (&sv)[CPW][2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int sg = 2 * t + h;
            const int g = sg / p.spg;
            const bool ends = ((sg + 1) % p.spg == 0) && g < p.NG;
#pragma unroll
            for (int c = 0; c < CPW; ++c)
                sv[c][h] = (ends && cval[c]) ? static_cast<uint32_t>(sp[c][g * 16]) : 0u;
        }
    };

    uint4 wb[kPF][CPW];
    uint32_t sb[kPF][CPW][2];
#pragma unroll
    for (int s = 0; s < kPF; ++s) {
        const int t = t0 + s;
#pragma unroll
        for (int c = 0; c < CPW; ++c)
            wb[s][c] = (t < t1 && cval[c]) ? wp[c][static_cast<int64_t>(t) * 64] : make_uint4(0, 0, 0, 0);
        if (t < t1) load_scales(t, sb[s]);
    }

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

    int chunk_t0 = t0;
    const int rowq = 4 * (lane >> 4);  // first output row of this lane inside a 16-row tile
    const int colq = lane & 15;

    for (int tb = t0; tb < t1; tb += kPF) {
#pragma unroll
        for (int s = 0; s < kPF; ++s) {
            const int t = tb + s;
            if (t >= t1) break;
            if (((t - t0) % Cfg::kTC) == 0) {
                // Stage A[:, t*128 : (t+tc)*128) into LDS; rows >= M and K >= K are zero.
                chunk_t0 = t;
                const int tc = min(Cfg::kTC, t1 - t);
                const int upr = tc * 8;  // 16-byte units per row
                __syncthreads();
                for (int u = threadIdx.x; u < Cfg::kRows * upr; u += kThreads) {
                    const int r = u / upr;
                    const int cu = u - r * upr;
                    const int64_t k = static_cast<int64_t>(t) * 128 + cu * 16;
                    uint4 v = make_uint4(0, 0, 0, 0);
                    if (r < p.M && k < p.K) v = *reinterpret_cast<const uint4*>(p.A + r * p.lda + k);
                    *reinterpret_cast<uint4*>(lds + r * Cfg::kLStride + cu * 16) = v;
                }
                __syncthreads();
            }
            uint4 wc[CPW];
            uint32_t sc[CPW][2];
#pragma unroll
            for (int c = 0; c < CPW; ++c) {
                wc[c] = wb[s][c];
                sc[c][0] = sb[s][c][0];
                sc[c][1] = sb[s][c][1];
            }
            const int tn = t + kPF;
            if (tn < t1) {
#pragma unroll
                for (int c = 0; c < CPW; ++c)
                    wb[s][c] = cval[c] ? wp[c][static_cast<int64_t>(tn) * 64] : make_uint4(0, 0, 0, 0);
                load_scales(tn, sb[s]);
            }
            v4i b[CPW][2];
#pragma unroll
            for (int c = 0; c < CPW; ++c) unpack_tile_lane(wc[c], b[c][0], b[c][1]);
            const int8_t* arow = lds + colq * Cfg::kLStride + (t - chunk_t0) * 128 + (lane >> 4) * 16;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const v4i a = *reinterpret_cast<const v4i*>(arow + mt * 16 * Cfg::kLStride + h * 64);
#pragma unroll
                    for (int c = 0; c < CPW; ++c) P[mt][c] = mfma16(a, b[c][h], P[mt][c]);
                }
                const int sg = 2 * t + h;
                const int g = sg / p.spg;
                if (((sg + 1) % p.spg) == 0 && g < p.NG) {
#pragma unroll
                    for (int c = 0; c < CPW; ++c) {
                        const float ws = scale_to_f32<SBF16>(sc[c][h]);
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) {
                            if constexpr (DUMP) {
                                const int col = (nbw + c) * 16 + colq;
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

    if (p.ksplit == 1) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = mt * 16 + rowq + i;
                if (row >= p.M) continue;
                const float ts = bf16_bits_to_f32(p.a_scale[row]) * 0.0625f;
#pragma unroll
                for (int c = 0; c < CPW; ++c) {
                    const int col = (nbw + c) * 16 + colq;
                    if (col < p.N) p.Y[row * p.ldy + col] = static_cast<uint16_t>(f32_to_bf16_bits(acc[mt][c][i] * ts));
                }
            }
        }
        return;
    }

    // Split-K: publish this split's partial, last arrival reduces in split order.
    float* mypart = p.part + static_cast<int64_t>(blockIdx.y) * p.M * p.N;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = mt * 16 + rowq + i;
            if (row >= p.M) continue;
#pragma unroll
            for (int c = 0; c < CPW; ++c) {
                const int col = (nbw + c) * 16 + colq;
                if (col < p.N) mypart[static_cast<int64_t>(row) * p.N + col] = acc[mt][c][i];
            }
        }
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = atomicAdd(p.cnt + blockIdx.x, 1u);
        s_last = (prev == static_cast<uint32_t>(p.ksplit - 1)) ? 1u : 0u;
    }
    __syncthreads();
    if (s_last == 0u) return;
    __threadfence();
    constexpr int kCols = kWaves * CPW * 16;
    const int col0 = blockIdx.x * kCols;
    for (int idx = threadIdx.x; idx < p.M * kCols; idx += kThreads) {
        const int row = idx / kCols;
        const int col = col0 + (idx - row * kCols);
        if (col >= p.N) continue;
        const int64_t off = static_cast<int64_t>(row) * p.N + col;
        float sum = 0.0f;
        for (int ks = 0; ks < p.ksplit; ++ks) sum += __builtin_nontemporal_load(p.part + static_cast<int64_t>(ks) * p.M * p.N + off);
        const float ts = bf16_bits_to_f32(p.a_scale[row]) * 0.0625f;
        p.Y[row * p.ldy + col] = static_cast<uint16_t>(f32_to_bf16_bits(sum * ts));
    }
    if (threadIdx.x == 0) p.cnt[blockIdx.x] = 0u;
}

struct DecodePlan {
    int MT, CPW, ksplit, tps;
    int64_t ncg;
};

int gcd_i(int a, int b) { while (b) { int t = a % b; a = b; b = t; } return a; }

DecodePlan plan_decode(int64_t M, int64_t N, int64_t K, int64_t group) {
    DecodePlan pl{};
    pl.MT = static_cast<int>(geom::ceil_div(M, 16));
    pl.CPW = 1;
    const int64_t NB = geom::col_blocks(N);
    pl.ncg = geom::ceil_div(NB, kWaves * pl.CPW);
    const int KT = static_cast<int>(geom::k_tiles(K, group));
    const int spg = static_cast<int>(group / 64);
    // Split boundaries must fall on both tile (2 slabs) and group boundaries.
    const int unit_slabs = 2 * spg / gcd_i(2, spg);
    const int unit = unit_slabs / 2;
    const int units = (KT + unit - 1) / unit;
    const int64_t target = 4 * static_cast<int64_t>(device_cu_count());
    int ks = static_cast<int>(std::max<int64_t>(1, (target + pl.ncg - 1) / pl.ncg));
    ks = std::min(ks, units);
    if (pl.ncg > kMaxCounters) ks = 1;  // wide N has enough column groups without split-K
    const int ups = (units + ks - 1) / ks;
    pl.tps = ups * unit;
    pl.ksplit = (KT + pl.tps - 1) / pl.tps;
    return pl;
}

template <int MT, bool SBF16, bool DUMP>
hipError_t launch_mt(const DecodeParams& p, const DecodePlan& pl, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(pl.ncg), static_cast<unsigned>(pl.ksplit));
    gemm_decode_kernel<MT, 1, SBF16, DUMP><<<grid, dim3(kThreads), 0, stream>>>(p);
    return hipGetLastError();
}

template <bool SBF16, bool DUMP>
hipError_t launch_sd(const DecodeParams& p, const DecodePlan& pl, hipStream_t stream) {
    switch (pl.MT) {
        case 1: return launch_mt<1, SBF16, DUMP>(p, pl, stream);
        case 2: return launch_mt<2, SBF16, DUMP>(p, pl, stream);
        case 3: return launch_mt<3, SBF16, DUMP>(p, pl, stream);
        default: return launch_mt<4, SBF16, DUMP>(p, pl, stream);
    }
}

}  // namespace

int64_t decode_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group) {
    const DecodePlan pl = plan_decode(M, N, K, group);
    if (pl.ksplit <= 1) return 0;
    return kCounterBytes + static_cast<int64_t>(pl.ksplit) * M * N * 4;
}

hipError_t launch_gemm_decode(const GemmArgs& a, hipStream_t stream) {
    const DecodePlan pl = plan_decode(a.M, a.N, a.K, a.group);
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
    p.tps = pl.tps;
    p.ksplit = pl.ksplit;
    if (pl.ksplit > 1) {
        p.cnt = reinterpret_cast<uint32_t*>(a.workspace);
        p.part = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(a.workspace) + kCounterBytes);
    }
    const bool dump = a.partials != nullptr;
    if (a.scale_bf16) return dump ? launch_sd<true, true>(p, pl, stream) : launch_sd<true, false>(p, pl, stream);
    return dump ? launch_sd<false, true>(p, pl, stream) : launch_sd<false, false>(p, pl, stream);
}

}  // namespace w4a8
