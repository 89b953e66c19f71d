// Prefill-shaped W4A8 GEMM (M > 64): int8 MFMA bound.
//
// Same arithmetic as the decode path (see gemm_decode.hip): exact int32 per
// group, fp32 fold with the group scale, token scale at the end.
//
// Tiling: a 256-thread workgroup computes a BM x BN = 128 x 128 output tile;
// its four waves form a 2 x 2 grid of 64 x 64 wave tiles, each 2 x 2
// v_mfma_i32_32x32x32_i8 blocks.  The K loop walks 128-K steps (one repacked
// weight tile row).  Each step the workgroup stages 128 x 128 int8
// activations and 128 columns x 128 K of weights in LDS; the weights arrive as
// packed int4 (8 KB) and are unpacked once on the way into LDS, so the four
// waves share the unpack.  The next step's global loads are issued into
// registers before the current step's MFMAs (register double buffering).
#include "common.h"
#include "kgeom.h"
#include "launch.h"

namespace w4a8 {
namespace {

constexpr int kThreads = 256;
constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kLS = 128 + 16;  // LDS row stride in bytes (+16 against bank conflicts)

struct PrefillParams {
    const int8_t* A;
    int64_t lda;
    const uint16_t* a_scale;
    const uint4* W;
    const uint16_t* S;
    uint16_t* Y;
    int64_t ldy;
    int32_t* P;
    int M, N, K;
    int KT, NG, NB;
    int group;
};

template <bool SBF16, bool DUMP>
__global__ __launch_bounds__(kThreads) void gemm_prefill_kernel(const PrefillParams p) {
    __shared__ __attribute__((aligned(16))) int8_t la[kBM * kLS];
    __shared__ __attribute__((aligned(16))) int8_t lb[kBN * kLS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;  // wave row (0..1)
    const int wn = wave & 1;   // wave col (0..1)
    const int m0 = blockIdx.y * kBM;
    const int n0 = blockIdx.x * kBN;
    const int nb0 = n0 / 16;

    // Global -> register staging of one K step.
    uint4 ra[4];
    uint4 rb[2];
    auto load_step = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = i * kThreads + tid;
            const int r = c >> 3;
            const int cu = c & 7;
            const int row = m0 + r;
            const int64_t k = static_cast<int64_t>(kt) * 128 + cu * 16;
            ra[i] = (row < p.M && k < p.K) ? *reinterpret_cast<const uint4*>(p.A + row * p.lda + k)
                                           : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = i * kThreads + tid;
            const int j = c >> 6;
            const int ll = c & 63;
            const int nb = nb0 + j;
            rb[i] = (nb < p.NB) ? p.W[(static_cast<int64_t>(nb) * p.KT + kt) * 64 + ll] : make_uint4(0, 0, 0, 0);
        }
    };
    auto store_step = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = i * kThreads + tid;
            *reinterpret_cast<uint4*>(la + (c >> 3) * kLS + (c & 7) * 16) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = i * kThreads + tid;
            const int j = c >> 6;
            const int ll = c & 63;
            v4i s0, s1;
            unpack_tile_lane(rb[i], s0, s1);
            int8_t* dst = lb + (j * 16 + (ll & 15)) * kLS + (ll >> 4) * 16;
            *reinterpret_cast<v4i*>(dst) = s0;
            *reinterpret_cast<v4i*>(dst + 64) = s1;
        }
    };

    // Scales of this lane's two columns for the groups ending in step kt.
    const int colw = n0 + wn * 64 + (lane & 31);
    uint32_t sc[2][2];
    auto load_scales = [&](int kt, uint32_t (&s)[2][2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int kend = kt * 128 + (h + 1) * 64;
            const int g = (kend - 1) / p.group;
            const bool ends = (kend % p.group) == 0 && g < p.NG;
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                const int col = colw + cb * 32;
                const int nb = col >> 4;
                s[cb][h] = (ends && nb < p.NB) ? static_cast<uint32_t>(p.S[(static_cast<int64_t>(nb) * p.NG + g) * 16 + (col & 15)]) : 0u;
            }
        }
    };

    v16i P[2][2];
    float acc[2][2][16];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                P[a][b][i] = 0;
                acc[a][b][i] = 0.0f;
            }
        }

    load_step(0);
    load_scales(0, sc);
    store_step();
    __syncthreads();

    const int8_t* abase = la + (wm * 64 + (lane & 31)) * kLS + (lane >> 5) * 16;
    const int8_t* bbase = lb + (wn * 64 + (lane & 31)) * kLS + (lane >> 5) * 16;

    for (int kt = 0; kt < p.KT; ++kt) {
        uint32_t scn[2][2];
        const bool more = (kt + 1) < p.KT;
        if (more) {
            load_step(kt + 1);
            load_scales(kt + 1, scn);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            v4i av[2], bv[2];
#pragma unroll
            for (int r = 0; r < 2; ++r) av[r] = *reinterpret_cast<const v4i*>(abase + r * 32 * kLS + s * 32);
#pragma unroll
            for (int c = 0; c < 2; ++c) bv[c] = *reinterpret_cast<const v4i*>(bbase + c * 32 * kLS + s * 32);
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int c = 0; c < 2; ++c) P[r][c] = mfma32(av[r], bv[c], P[r][c]);
            if (s & 1) {
                const int h = s >> 1;
                const int kend = kt * 128 + (h + 1) * 64;
                const int g = (kend - 1) / p.group;
                if ((kend % p.group) == 0 && g < p.NG) {
#pragma unroll
                    for (int c = 0; c < 2; ++c) {
                        const float ws = scale_to_f32<SBF16>(sc[c][h]);
#pragma unroll
                        for (int r = 0; r < 2; ++r) {
                            if constexpr (DUMP) {
                                const int col = colw + c * 32;
#pragma unroll
                                for (int i = 0; i < 16; ++i) {
                                    const int row = m0 + wm * 64 + r * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
                                    if (row < p.M && col < p.N)
                                        p.P[(static_cast<int64_t>(g) * p.M + row) * p.N + col] = P[r][c][i] >> 4;
                                }
                            }
#pragma unroll
                            for (int i = 0; i < 16; ++i) {
                                acc[r][c][i] += static_cast<float>(P[r][c][i]) * ws;
                                P[r][c][i] = 0;
                            }
                        }
                    }
                }
            }
        }
        if (more) {
            __syncthreads();
            store_step();
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int h = 0; h < 2; ++h) sc[c][h] = scn[c][h];
            __syncthreads();
        }
    }

#pragma unroll
    for (int r = 0; r < 2; ++r) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = m0 + wm * 64 + r * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
            if (row >= p.M) continue;
            const float ts = bf16_bits_to_f32(p.a_scale[row]) * 0.0625f;
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int col = colw + c * 32;
                if (col < p.N) p.Y[row * p.ldy + col] = static_cast<uint16_t>(f32_to_bf16_bits(acc[r][c][i] * ts));
            }
        }
    }
}

template <bool SBF16, bool DUMP>
hipError_t launch(const PrefillParams& p, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(geom::ceil_div(p.N, kBN)), static_cast<unsigned>(geom::ceil_div(p.M, kBM)));
    gemm_prefill_kernel<SBF16, DUMP><<<grid, dim3(kThreads), 0, stream>>>(p);
    return hipGetLastError();
}

}  // namespace

int64_t prefill_workspace_bytes(int64_t, int64_t, int64_t, int64_t) { return 0; }

hipError_t launch_gemm_prefill(const GemmArgs& a, hipStream_t stream) {
    PrefillParams p{};
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
    p.group = static_cast<int>(a.group);
    const bool dump = a.partials != nullptr;
    if (a.scale_bf16) return dump ? launch<true, true>(p, stream) : launch<true, false>(p, stream);
    return dump ? launch<false, true>(p, stream) : launch<false, false>(p, stream);
}

}  // namespace w4a8
