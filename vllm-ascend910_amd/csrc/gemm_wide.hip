// Decode-shaped W4A8 GEMM for 16 < M <= 64 rows on wide N, the activations
// shared through LDS.
//
// Same arithmetic as gemm_decode.hip (exact int32 per group on
// v_mfma_i32_16x16x64_i8, fp32 fold with the group scale, token scale at the
// end).  The decode kernel gives every wave all rows and its own K range, so
// every workgroup streams the whole activation block from L2 for its few
// column blocks: at 64 rows on gate_up that is twice the weight bytes.  Here a
// workgroup of kWN column waves covers kWN * kCPW column blocks and walks all
// of K; its waves share each 64-row activation tile, staged once into LDS
// (double-buffered, one barrier per tile) and read from there as MFMA
// operands, while the weights stream straight to registers in a 2-deep ring
// as in the decode kernel.  The accumulation order per output is the decode
// kernel's with one K wave, so the sums are bit-identical to it.  (Measured
// on the QwQ-32B shapes: on narrow N -- a few dozen workgroups -- adding K
// splits reduced through LDS did not reach the decode kernel's row groups.)
#include <type_traits>

#include "common.h"
#include "kgeom.h"
#include "launch.h"

namespace w4a8 {
namespace {

constexpr int kMT = 4;                 // 16-row tiles: 64 rows
constexpr int kD = 2;                  // weight ring depth (tiles)
constexpr int kALS = 128 + 16;         // LDS row stride of a staged activation tile (bytes)
constexpr int kATile = 16 * kMT * kALS;  // one staged tile
constexpr uint32_t kOOBW = 0x80000000u;

struct WideParams {
    const int8_t* A;
    int64_t lda;
    const uint16_t* a_scale;
    const uint4* W;
    const uint16_t* S;
    uint16_t* Y;
    int64_t ldy;
    int32_t* P;        // optional partial dump [NG, M, N]
    int M, N, KT, NG, NB;
    int up_nb;         // SWIGLU: column blocks per half
    int nslab, spg, gshift;
    uint32_t a_bytes, w_bytes, s_bytes;
};

// GM: the group modes of gemm_decode.hip (0: stride 64, 3: stride 128,
// 1: stride 128 * 2^gshift, 2: any other stride).
// kWN column waves, kCPW 16-column blocks per wave.
template <int kWN, int kCPW, int GM, bool SBF16, bool DUMP, bool SWIGLU>
__global__ __launch_bounds__(64 * kWN) void gemm_wide_kernel(const WideParams p) {
    static_assert(!(SWIGLU && DUMP), "the SwiGLU variant dumps nothing");
    constexpr int CG = SWIGLU ? kCPW / 2 : kCPW;   // output column blocks per wave
    constexpr int NS = (GM == 1 || GM == 3) ? 1 : 2;
    // two staged activation tiles
    __shared__ __attribute__((aligned(16))) int8_t la[2][kATile];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave;
    const int rowq = 4 * (lane >> 4);
    const int colq = lane & 15;

    const int nb0 = (static_cast<int>(blockIdx.x) * kWN + wn) * CG;
    auto block_of = [&](int c) { return (SWIGLU && c >= CG) ? nb0 + (c - CG) + p.up_nb : nb0 + c; };

    // All of K: tiles [0, KT).
    const int ta = 0, tb = p.KT, nit = p.KT;

    uint32_t wo[kCPW], so[kCPW];
#pragma unroll
    for (int c = 0; c < kCPW; ++c) {
        const uint32_t nb = static_cast<uint32_t>(min(block_of(c), p.NB - 1));
        wo[c] = nb * static_cast<uint32_t>(p.KT) * 1024u + lane * 16u;
        so[c] = (nb * static_cast<uint32_t>(p.NG) * 16u + colq) * 2u;
    }
    // Staging: 64 rows x 128 K = 512 units of 16 bytes, NU per lane; rows
    // past M read zero.
    constexpr int NU = 512 / (64 * kWN);
    static_assert(NU * 64 * kWN == 512, "kWN must divide 8");
    uint32_t sg[NU];
    int sl[NU];
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        const int u = lane + 64 * (wn + kWN * j);
        const int r = u >> 3, c16 = (u & 7) * 16;
        sg[j] = r < p.M ? static_cast<uint32_t>(r) * static_cast<uint32_t>(p.lda) + c16 : kOOBW;
        sl[j] = r * kALS + c16;
    }
    auto gend = [&](int t, int h) -> int {
        int g;
        if constexpr (GM == 0) g = 2 * t + h;
        else if constexpr (GM == 3) g = t;
        else if constexpr (GM == 1) g = t >> p.gshift;
        else g = (2 * t + h) / p.spg;
        return min(g, p.NG - 1);
    };

    uint4 ra[2][NU];
    auto stage_load = [&](int t, uint4 (&r)[NU]) {
        // tiles past the end stage the last tile again (nothing reads them)
        const auto rs = make_rsrc_at(p.A, static_cast<uint32_t>(min(t, p.KT - 1)) * 128u, p.a_bytes);
#pragma unroll
        for (int j = 0; j < NU; ++j) r[j] = buf_load16(rs, sg[j]);
    };
    auto stage_store = [&](int buf, const uint4 (&r)[NU]) {
#pragma unroll
        for (int j = 0; j < NU; ++j) *reinterpret_cast<uint4*>(&la[buf][sl[j]]) = r[j];
    };

    uint4 wb[kD][kCPW];
    uint32_t sb[kD][kCPW][NS];
    auto load_slot = [&](int s, int t) {
        const auto rw = make_rsrc_at(p.W, static_cast<uint32_t>(min(t, p.KT - 1)) * 1024u, t < tb ? p.w_bytes : 0u);
#pragma unroll
        for (int c = 0; c < kCPW; ++c) wb[s][c] = buf_load16(rw, wo[c]);
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            const auto rs = make_rsrc_at(p.S, static_cast<uint32_t>(gend(min(t, p.KT - 1), j)) * 32u, p.s_bytes);
#pragma unroll
            for (int c = 0; c < kCPW; ++c) sb[s][c][j] = buf_load_u16(rs, so[c]);
        }
    };

    float acc[kMT][kCPW][4];
    v4i P[kMT][kCPW];
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
        for (int c = 0; c < kCPW; ++c) {
            P[mt][c] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[mt][c][i] = 0.0f;
        }

    auto fold = [&](int g, bool own, const uint32_t (&sc)[kCPW][NS], int j) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < kCPW; ++c) {
            const float ws = scale_to_f32<SBF16>(sc[c][j]);
#pragma unroll
            for (int mt = 0; mt < kMT; ++mt) {
                if constexpr (DUMP) {
                    const int col = block_of(c) * 16 + colq;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int row = mt * 16 + rowq + i;
                        if (own && row < p.M && col < p.N && g < p.NG)
                            p.P[(static_cast<int64_t>(g) * p.M + row) * p.N + col] = P[mt][c][i] >> 4;
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mt][c][i] += static_cast<float>(P[mt][c][i]) * ws;
                if constexpr (GM == 1 || GM == 2) P[mt][c] = v4i{0, 0, 0, 0};
            }
        }
    };

    // ---- prologue: tile ta staged in buffer 0, ta+1 in registers, the ring in flight
    stage_load(ta, ra[0]);
    stage_load(ta + 1, ra[1]);
#pragma unroll
    for (int s = 0; s < kD; ++s) load_slot(s, ta + s);
    stage_store(0, ra[0]);
    __syncthreads();

    // One tile: u = iteration parity (the staging registers and the ring slot).
    auto step = [&](int i, int u) __attribute__((always_inline)) {
        const int t = ta + i;
        stage_load(t + 2, ra[u]);
        uint32_t sc[kCPW][NS];
#pragma unroll
        for (int c = 0; c < kCPW; ++c)
#pragma unroll
            for (int j = 0; j < NS; ++j) sc[c][j] = sb[u][c][j];
        v4i b[kCPW][2];
#pragma unroll
        for (int c = 0; c < kCPW; ++c) unpack_tile_lane(wb[u][c], b[c][0], b[c][1]);
        load_slot(u, t + kD);
        const int8_t* ab = &la[u][0] + colq * kALS + (lane >> 4) * 16;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const bool fresh = GM == 0 || (GM == 3 && h == 0);
#pragma unroll
            for (int mt = 0; mt < kMT; ++mt) {
                const v4i a = *reinterpret_cast<const v4i*>(ab + mt * 16 * kALS + h * 64);
#pragma unroll
                for (int c = 0; c < kCPW; ++c) P[mt][c] = mfma16(a, b[c][h], fresh ? v4i{0, 0, 0, 0} : P[mt][c]);
            }
            if constexpr (GM == 0) {
                fold(2 * t + h, t < tb, sc, h);
            } else if constexpr (GM == 3) {
                if (h == 1) fold(t, t < tb, sc, 0);
            } else if constexpr (GM == 1) {
                if (h == 1 && (((t + 1) & ((1 << p.gshift) - 1)) == 0 || t == p.KT - 1))
                    fold(t >> p.gshift, t < tb, sc, 0);
            } else {
                const int sgi = 2 * t + h;
                if (sgi < p.nslab && (((sgi + 1) % p.spg) == 0 || sgi == p.nslab - 1))
                    fold(sgi / p.spg, t < tb, sc, h);
            }
        }
        // tile t+1 into the other buffer (free: every wave finished tile t-1)
        stage_store(u ^ 1, ra[u ^ 1]);
        __syncthreads();
    };
    int i = 0;
    for (; i + 2 <= nit; i += 2) {
        step(i, 0);
        step(i + 1, 1);
    }
    if (i < nit) step(i, 0);

    // ---- epilogue: token scale, bf16 (or the SwiGLU pair)
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int row = mt * 16 + rowq + q;
            if (row >= p.M) continue;
            const float ts = bf16_bits_to_f32(p.a_scale[row]) * 0.0625f;
            if constexpr (SWIGLU) {
#pragma unroll
                for (int c = 0; c < CG; ++c) {
                    const int col = block_of(c) * 16 + colq;
                    if (col < p.up_nb * 16)
                        p.Y[static_cast<int64_t>(row) * p.ldy + col] =
                            static_cast<uint16_t>(swiglu_bf16_bits(acc[mt][c][q] * ts, acc[mt][c + CG][q] * ts));
                }
            } else {
#pragma unroll
                for (int c = 0; c < kCPW; ++c) {
                    const int col = block_of(c) * 16 + colq;
                    if (col < p.N)
                        p.Y[static_cast<int64_t>(row) * p.ldy + col] =
                            static_cast<uint16_t>(f32_to_bf16_bits(acc[mt][c][q] * ts));
                }
            }
        }
}

int group_mode_of(int spg) {
    if (spg == 1) return 0;
    if (spg == 2) return 3;
    if (spg % 2 == 0 && ((spg / 2) & (spg / 2 - 1)) == 0) return 1;
    return 2;
}

constexpr int kWaves = 4;   // column waves per workgroup
constexpr int kBlocks = 2;  // column blocks per wave

template <int GM, bool DUMP, bool SWIGLU>
hipError_t launch_g(const WideParams& p, int cgroups, bool sbf16, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(cgroups)), block(64 * kWaves);
    if (sbf16) gemm_wide_kernel<kWaves, kBlocks, GM, true, DUMP, SWIGLU><<<grid, block, 0, s>>>(p);
    else gemm_wide_kernel<kWaves, kBlocks, GM, false, DUMP, SWIGLU><<<grid, block, 0, s>>>(p);
    return hipGetLastError();
}

template <bool DUMP, bool SWIGLU>
hipError_t launch_gm(const WideParams& p, int cgroups, bool sbf16, hipStream_t s) {
    switch (group_mode_of(p.spg)) {
        case 0: return launch_g<0, DUMP, SWIGLU>(p, cgroups, sbf16, s);
        case 1: return launch_g<1, DUMP, SWIGLU>(p, cgroups, sbf16, s);
        case 3: return launch_g<3, DUMP, SWIGLU>(p, cgroups, sbf16, s);
        default: return launch_g<2, DUMP, SWIGLU>(p, cgroups, sbf16, s);
    }
}

}  // namespace

hipError_t launch_gemm_wide(const GemmArgs& a, hipStream_t stream) {
    if (a.M <= 0 || a.M > 16 * kMT) return hipErrorInvalidValue;
    WideParams p{};
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
    p.KT = static_cast<int>(geom::k_tiles(a.K, a.group));
    p.NG = static_cast<int>(geom::num_groups(a.K, a.group));
    p.NB = static_cast<int>(geom::col_blocks(a.N));
    p.up_nb = a.swiglu ? static_cast<int>(a.N / 2 / geom::kTileN) : 0;
    p.nslab = static_cast<int>(geom::kpad(a.K, a.group) / 64);
    p.spg = static_cast<int>(geom::group_stride(a.group) / 64);
    p.gshift = 0;
    while ((2 << p.gshift) < p.spg) ++p.gshift;
    p.a_bytes = static_cast<uint32_t>((a.M - 1) * a.lda + geom::kpad(a.K, a.group));
    p.w_bytes = static_cast<uint32_t>(p.NB * static_cast<int64_t>(p.KT) * geom::kTileBytes);
    p.s_bytes = static_cast<uint32_t>(p.NB * static_cast<int64_t>(p.NG) * 16 * 2);
    const int per_wg = kWaves * kBlocks;
    const int64_t cg = a.swiglu ? geom::ceil_div(p.up_nb, per_wg / 2) : geom::ceil_div(p.NB, per_wg);
    const int c = static_cast<int>(cg);
    if (a.swiglu) return launch_gm<false, true>(p, c, a.scale_bf16, stream);
    return a.partials ? launch_gm<true, false>(p, c, a.scale_bf16, stream)
                      : launch_gm<false, false>(p, c, a.scale_bf16, stream);
}

}  // namespace w4a8
