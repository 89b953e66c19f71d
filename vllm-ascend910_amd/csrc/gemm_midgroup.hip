// Mid-group W4A8 GEMM on the reference's compat tensors (gfx950).
//
// Computes the reference's `midgroup_w4a8_gemm` (host
// npu_ops/host/midgroup_w4a8_gemm.cpp:45-140, kernel
// npu_ops/kernel/midgroup_w4a8_gemm.inc; CPU definition
// int4_cube_lab/host/gemm_ref.cpp:199-240, ReferenceMidGroupGemm):
//   I_g[m,n] = sum_{k in g} A[m,k] * (W[n,k] - wz[g,n])          (int32, exact)
//   y[m,n]   = bf16( sum_g (float(I_g) * ws[g,n]) * as[g,m] )     (fp32, group order)
// where A = 16*hi + lo + 8 comes from the MSD planes of `midgroup_quant_a` and
// W, wz, ws, as are the reference's tensors as stored -- nothing is repacked.
//
// Operand loading.  The contraction is invariant under any permutation of K
// applied to both operands, which lets every lane read contiguous bytes of the
// row-major packed tensors: in a 128-K tile, lane l (column or row l % 16,
// quad q = l / 16) takes K [32q, 32q + 32) -- 16 bytes of w_q, a_hi and a_lo
// each -- as its chunk of slab 0 (first 16 codes) and slab 1 (next 16).  Inside a
// chunk both operands are split into even and odd codes the same way: the
// weight's nibbles move into the high half of each byte (16*W, as in the
// per-token kernels) and each activation byte is rebuilt from its two nibbles
// ((hi << 4) | (lo ^ 8)), so v_mfma_i32_16x16x64_i8 accumulates 16 * sum A*W.
// The zero point enters through the rank-1 identity
//   sum A*(W - wz) = sum A*W + wz * a_ksum     (a_ksum = -sum A, as stored)
// whose int32 result is exact, then the fold follows the reference's fp32
// order: (float(I) * ws) * as, added to the accumulator group by group.
//
// Work split as in the decode kernel: a workgroup owns CPW column blocks of 16
// and a block of 16*MT rows (grid.y walks row blocks); its KW waves split K
// and add their exact int32 group sums into LDS, after which the workgroup
// folds the groups in order (in chunks of groups when their sums exceed the
// LDS), or a single wave walks all of K (prefill shapes: 64 x 64 tiles, K
// split only while the grid is small).  The
// activation scales and ksums of the workgroup's rows, and the weight scales
// and zero points of its columns, are staged in LDS once.  All global reads are
// raw buffer loads; rows and columns past the tensors, and the K tail past
// kpad, read as zero.
#include <algorithm>

#include "common.h"
#include "kgeom.h"
#include "launch.h"

namespace w4a8 {
namespace {

constexpr uint32_t kOOBm = 0x80000000u;
constexpr size_t kMidLdsLimit = 64 * 1024;
// The int32 group sums of the tile-granular K split may take the workgroup's
// LDS past the 64 KiB a launch gets by default (down_proj at one 16-row tile:
// 27 groups of 16 x 32 sums), up to this much (the attribute is set once per
// kernel).
constexpr size_t kMidLdsIsum = 128 * 1024;

struct MidParams {
    const uint8_t* a_hi;
    const uint8_t* a_lo;
    const uint16_t* a_scale;   // bf16 [G, ld_as]
    const int32_t* a_ksum;     // int32 [G, ld_as]
    const uint8_t* w_q;        // [N, kpad/2]
    const uint16_t* w_scale;   // bf16 [G, N]
    const uint16_t* w_zero;    // bf16 [G, N] or null
    uint16_t* Y;
    int32_t* P;                // optional [G, Ma, N]
    int64_t ldy;
    int Ma, ld_as, N, K;
    int kb;                    // packed row pitch (kpad / 2 bytes)
    int kpad, KT, NG, NB;
    int tpg;                   // 128-K tiles per group stride
    uint32_t a_bytes, w_bytes;
    bool isum;                 // K split over waves at tile granularity, int32 group sums in LDS
    int gchunk;                // isum: groups whose sums LDS holds at once (chunks of them, folded in turn)
    bool wtiles;               // w_q is w4a8_midgroup_tile_weights' layout (1 KB tiles), not [N, kpad/2]
};

// The weight's byte offset of lane (column col, quad q) in K tile 0, and the
// stride of one K tile: rows as stored ([N, kpad/2], 64 bytes a tile), or the
// tile layout ([col block][K tile][quad][column in block][16 bytes]: a
// block's tile is 1 KB contiguous -- the same bytes, one 16-byte load per lane
// either way).
__device__ __forceinline__ uint32_t mid_woff(const MidParams& p, int col, int q) {
    if (col >= p.N) return kOOBm;
    if (p.wtiles)
        return static_cast<uint32_t>(col >> 4) * static_cast<uint32_t>(p.KT) * 1024u +
               (16u * static_cast<uint32_t>(q) + static_cast<uint32_t>(col & 15)) * 16u;
    return static_cast<uint32_t>(col) * static_cast<uint32_t>(p.kb) + 16u * static_cast<uint32_t>(q);
}
__device__ __forceinline__ uint32_t mid_wstep(const MidParams& p) { return p.wtiles ? 1024u : 64u; }

template <int MT, int CPW, int KWMAX, int D, bool ASYM, bool DUMP>
__global__ __launch_bounds__(64 * KWMAX) void gemm_midgroup_kernel(const MidParams p) {
    constexpr int R = 16 * MT;
    constexpr int C = 16 * CPW;
    extern __shared__ float smem[];
    // [NG][R] activation scales (fp32), [NG][R] ksums, [NG][C] weight scales,
    // [NG][C] zero points, then the K-split reduction buffer: [kw][R][C] fp32
    // wave sums, or with p.isum the int32 group sums [NG][R][C].
    float* s_as = smem;
    int* s_ak = reinterpret_cast<int*>(s_as + p.NG * R);
    float* s_ws = reinterpret_cast<float*>(s_ak + p.NG * R);
    float* s_wz = s_ws + p.NG * C;
    float* red = s_wz + p.NG * C;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kw = blockDim.x >> 6;
    const int nb0 = blockIdx.x * CPW;
    const int m0 = blockIdx.y * R;
    const int q = lane >> 4;
    const int rowq = 4 * q;
    const int colq = lane & 15;

    for (int e = threadIdx.x; e < p.NG * R; e += blockDim.x) {
        const int g = e / R, r = e - g * R;
        const int row = m0 + r;
        const bool ok = row < p.Ma;
        s_as[e] = ok ? bf16_bits_to_f32(p.a_scale[static_cast<int64_t>(g) * p.ld_as + row]) : 0.0f;
        s_ak[e] = ok ? p.a_ksum[static_cast<int64_t>(g) * p.ld_as + row] : 0;
    }
    for (int e = threadIdx.x; e < p.NG * C; e += blockDim.x) {
        const int g = e / C, cc = e - g * C;
        const int col = nb0 * 16 + cc;
        const bool ok = col < p.N;
        s_ws[e] = ok ? bf16_bits_to_f32(p.w_scale[static_cast<int64_t>(g) * p.N + col]) : 0.0f;
        s_wz[e] = (ASYM && ok) ? bf16_bits_to_f32(p.w_zero[static_cast<int64_t>(g) * p.N + col]) : 0.0f;
    }

    // This wave's tile range [ta, tb).  p.isum: an even share of the tiles of
    // the current chunk of p.gchunk groups, groups split between waves meeting
    // in the int32 sums; otherwise one wave walks every group (the host
    // launches a single wave then).
    int ta = 0, tb = 0;
    auto share = [&](int T0, int T1) {
        ta = T0 + (wave * (T1 - T0)) / kw;
        tb = T0 + ((wave + 1) * (T1 - T0)) / kw;
    };
    const int gch = p.isum ? p.gchunk : p.NG;
    share(0, min(p.KT, gch * p.tpg));
    // [gch][R][C] int32 group sums, then (more than one chunk) the running
    // fp32 fold [R][C] of each output, carried from chunk to chunk
    int* const isum = reinterpret_cast<int*>(red);
    float* const accl = reinterpret_cast<float*>(isum + gch * R * C);
    if (p.isum)
        for (int e = threadIdx.x; e < gch * R * C; e += blockDim.x) isum[e] = 0;

    uint32_t wo[CPW], ao[MT];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const int col = (nb0 + c) * 16 + colq;
        wo[c] = mid_woff(p, col, q);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int row = m0 + mt * 16 + colq;
        ao[mt] = row < p.Ma ? static_cast<uint32_t>(row) * static_cast<uint32_t>(p.kb) + 16u * q : kOOBm;
    }

    uint4 wb[D][CPW];
    uint4 hb[D][MT], lb[D][MT];
    auto load_slot = [&](int s, int t) {
        // tiles past the wave's range read zero weights; in a last tile that
        // is half padding, the upper quads read zero weights
        const uint32_t base = static_cast<uint32_t>(min(t, p.KT - 1)) * 64u;
        const bool half = q >= 2 && (p.kpad - t * 128) < 128;
        const auto rw = make_rsrc_at(p.w_q, static_cast<uint32_t>(min(t, p.KT - 1)) * mid_wstep(p), t < tb ? p.w_bytes : 0u);
        const auto rh = make_rsrc_at(p.a_hi, base, p.a_bytes);
        const auto rl = make_rsrc_at(p.a_lo, base, p.a_bytes);
#pragma unroll
        for (int c = 0; c < CPW; ++c) wb[s][c] = buf_load16(rw, half ? kOOBm : wo[c]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            hb[s][mt] = buf_load16(rh, ao[mt]);
            lb[s][mt] = buf_load16(rl, ao[mt]);
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
    __syncthreads();   // LDS scales staged

    // p.isum: this wave's int32 sum of group g (sum A*W, exact) into the
    // group's LDS sums; the fold happens once every wave has added its share.
    auto flush = [&](int g) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < CPW; ++c)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    atomicAdd(&isum[(g * R + mt * 16 + rowq + i) * C + c * 16 + colq], P[mt][c][i] >> 4);
                P[mt][c] = v4i{0, 0, 0, 0};
            }
    };
    auto fold = [&](int g, bool own) __attribute__((always_inline)) {
        // the reference's separate roundings: no multiply-add contraction
#pragma clang fp contract(off)
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
            const float ws = s_ws[g * C + c * 16 + colq];
            const int wz = ASYM ? static_cast<int>(s_wz[g * C + c * 16 + colq]) : 0;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = mt * 16 + rowq + i;
                    const int I = (P[mt][c][i] >> 4) + (ASYM ? wz * s_ak[g * R + r] : 0);
                    if constexpr (DUMP) {
                        const int row = m0 + r, col = (nb0 + c) * 16 + colq;
                        if (own && row < p.Ma && col < p.N && g < p.NG)
                            p.P[(static_cast<int64_t>(g) * p.Ma + row) * p.N + col] = I;
                    }
                    const float t1 = static_cast<float>(I) * ws;
                    acc[mt][c][i] = acc[mt][c][i] + t1 * s_as[g * R + r];
                }
                P[mt][c] = v4i{0, 0, 0, 0};
            }
        }
    };

    // The wave's range [ta, tb); group g's sums go to chunk slot g - gbase.
    auto run = [&](int gbase) __attribute__((always_inline)) {
        if (tb <= ta) return;
#pragma unroll
        for (int s = 0; s < D; ++s) load_slot(s, ta + s);
        for (int t0 = ta; t0 < tb; t0 += D) {
#pragma unroll
            for (int s = 0; s < D; ++s) {
                const int t = t0 + s;
                if (t >= tb) break;
                v4i bw[CPW][2];
#pragma unroll
                for (int c = 0; c < CPW; ++c) {
                    const uint4 w = wb[s][c];
                    bw[c][0] = v4i{unpack_lo4(w.x), unpack_hi4(w.x), unpack_lo4(w.y), unpack_hi4(w.y)};
                    bw[c][1] = v4i{unpack_lo4(w.z), unpack_hi4(w.z), unpack_lo4(w.w), unpack_hi4(w.w)};
                }
                v4i av[MT][2];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const uint4 h = hb[s][mt], l = lb[s][mt];
                    int e[4], o[4];
                    act_pair(h.x, l.x, e[0], o[0]);
                    act_pair(h.y, l.y, e[1], o[1]);
                    act_pair(h.z, l.z, e[2], o[2]);
                    act_pair(h.w, l.w, e[3], o[3]);
                    av[mt][0] = v4i{e[0], o[0], e[1], o[1]};
                    av[mt][1] = v4i{e[2], o[2], e[3], o[3]};
                }
                load_slot(s, t + D);
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int c = 0; c < CPW; ++c) P[mt][c] = mfma16(av[mt][h], bw[c][h], P[mt][c]);
                if (p.isum) {
                    if ((t + 1) % p.tpg == 0 || t == p.KT - 1 || t == tb - 1) flush(t / p.tpg - gbase);
                } else if ((t + 1) % p.tpg == 0 || t == p.KT - 1) {
                    fold(t / p.tpg, true);
                }
            }
        }
    };

    if (p.isum) {
        // Chunk by chunk: every wave adds its share of the chunk's int32 group
        // sums, then the fold in group order, one output element per thread
        // and step (each element stays with one thread, so its running fold
        // needs no barrier of its own)
#pragma clang fp contract(off)
        for (int g0 = 0; g0 < p.NG; g0 += gch) {
            const int g1 = min(p.NG, g0 + gch);
            if (g0 > 0) {
                share(g0 * p.tpg, min(p.KT, g1 * p.tpg));
                for (int e = threadIdx.x; e < (g1 - g0) * R * C; e += blockDim.x) isum[e] = 0;
                __syncthreads();
            }
            run(g0);
            __syncthreads();
            const bool last = g1 == p.NG;
            for (int e = threadIdx.x; e < R * C; e += blockDim.x) {
                const int r = e / C, cc = e - r * C;
                const int row = m0 + r;
                const int col = nb0 * 16 + cc;
                if (row >= p.Ma || col >= p.N) continue;
                float a = g0 == 0 ? 0.0f : accl[e];
                for (int g = g0; g < g1; ++g) {
                    const int I = isum[((g - g0) * R + r) * C + cc] +
                                  (ASYM ? static_cast<int>(s_wz[g * C + cc]) * s_ak[g * R + r] : 0);
                    if constexpr (DUMP) p.P[(static_cast<int64_t>(g) * p.Ma + row) * p.N + col] = I;
                    const float t1 = static_cast<float>(I) * s_ws[g * C + cc];
                    a = a + t1 * s_as[g * R + r];
                }
                if (last) p.Y[static_cast<int64_t>(row) * p.ldy + col] = static_cast<uint16_t>(f32_to_bf16_bits(a));
                else accl[e] = a;
            }
            if (!last) __syncthreads();   // the chunk's sums are read before the next chunk clears them
        }
        return;
    }

    // one wave: every group folded in order in its registers
    run(0);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int c = 0; c < CPW; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = m0 + mt * 16 + rowq + i, col = (nb0 + c) * 16 + colq;
                if (row < p.Ma && col < p.N)
                    p.Y[static_cast<int64_t>(row) * p.ldy + col] = static_cast<uint16_t>(f32_to_bf16_bits(acc[mt][c][i]));
            }
}

// Decode rows (Ma <= 16) on wide N: four waves of two column blocks each
// share the activation planes, staged through LDS two tiles (4 KB) at a time,
// so a workgroup reads them once rather than once per wave (on gate_up the
// activation-plane loads were a third of the time).  No K split: every wave
// walks all of K and folds group by group, the one-wave order of
// gemm_midgroup_kernel, so the outputs are the same bits.
constexpr int kShWaves = 4;   // column waves per workgroup
constexpr int kShCPW = 2;     // column blocks per wave
constexpr int kShD = 4;       // weight ring depth (tiles)
constexpr int kShP = 4;       // activation steps in flight (registers)

template <bool ASYM, bool DUMP>
__global__ __launch_bounds__(64 * kShWaves) void gemm_midgroup_shared_kernel(const MidParams p) {
    constexpr int R = 16, CPW = kShCPW, C = 16 * CPW * kShWaves, D = kShD, P = kShP;
    static_assert(P % 2 == 0 && D == 4, "the unrolled step indexes the rings statically");
    extern __shared__ float smem[];
    // [NG][16] activation scales, [NG][16] ksums, [NG][128] weight scales,
    // [NG][128] zero points
    float* s_as = smem;
    int* s_ak = reinterpret_cast<int*>(s_as + p.NG * R);
    float* s_ws = reinterpret_cast<float*>(s_ak + p.NG * R);
    float* s_wz = s_ws + p.NG * C;
    // two steps of two tiles, each tile [plane][row][64 B]; thread tid stages
    // the 16 bytes at tid * 16 of a step
    __shared__ __attribute__((aligned(16))) uint8_t ring[2][4096];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nbw = blockIdx.x * (kShWaves * CPW);
    const int q = lane >> 4;
    const int rowq = 4 * q;
    const int colq = lane & 15;

    for (int e = tid; e < p.NG * R; e += blockDim.x) {
        const int g = e / R, r = e - g * R;
        const bool ok = r < p.Ma;
        s_as[e] = ok ? bf16_bits_to_f32(p.a_scale[static_cast<int64_t>(g) * p.ld_as + r]) : 0.0f;
        s_ak[e] = ok ? p.a_ksum[static_cast<int64_t>(g) * p.ld_as + r] : 0;
    }
    for (int e = tid; e < p.NG * C; e += blockDim.x) {
        const int g = e / C, cc = e - g * C;
        const int col = nbw * 16 + cc;
        const bool ok = col < p.N;
        s_ws[e] = ok ? bf16_bits_to_f32(p.w_scale[static_cast<int64_t>(g) * p.N + col]) : 0.0f;
        s_wz[e] = (ASYM && ok) ? bf16_bits_to_f32(p.w_zero[static_cast<int64_t>(g) * p.N + col]) : 0.0f;
    }

    uint32_t wo[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const int col = (nbw + wave * CPW + c) * 16 + colq;
        wo[c] = mid_woff(p, col, q);
    }
    uint4 wb[D][CPW];
    auto load_w = [&](int s, int t) {
        const bool half = q >= 2 && (p.kpad - t * 128) < 128;
        const auto rw = make_rsrc_at(p.w_q, static_cast<uint32_t>(min(t, p.KT - 1)) * mid_wstep(p), t < p.KT ? p.w_bytes : 0u);
#pragma unroll
        for (int c = 0; c < CPW; ++c) wb[s][c] = buf_load16(rw, half ? kOOBm : wo[c]);
    };
    // this thread's 16 staged bytes: tile tid >> 7 of the step, plane
    // (tid >> 6) & 1, row (tid >> 2) & 15, quad tid & 3
    const int sts = tid >> 7;
    const int srow = (tid >> 2) & 15;
    const uint8_t* splane = ((tid >> 6) & 1) ? p.a_lo : p.a_hi;
    const uint32_t soff = srow < p.Ma ? static_cast<uint32_t>(srow) * static_cast<uint32_t>(p.kb) + 16u * (tid & 3)
                                      : kOOBm;
    auto load_a = [&](int step) {
        const int t = 2 * step + sts;
        const auto r = make_rsrc_at(splane, static_cast<uint32_t>(min(t, p.KT - 1)) * 64u, t < p.KT ? p.a_bytes : 0u);
        return buf_load16(r, soff);
    };

    float acc[CPW][4];
    v4i Pm[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        Pm[c] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[c][i] = 0.0f;
    }
    auto fold = [&](int g) __attribute__((always_inline)) {
        // the reference's separate roundings: no multiply-add contraction
#pragma clang fp contract(off)
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
            const int cw = (wave * CPW + c) * 16 + colq;
            const float ws = s_ws[g * C + cw];
            const int wz = ASYM ? static_cast<int>(s_wz[g * C + cw]) : 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = rowq + i;
                const int I = (Pm[c][i] >> 4) + (ASYM ? wz * s_ak[g * R + r] : 0);
                if constexpr (DUMP) {
                    const int col = nbw * 16 + cw;
                    if (r < p.Ma && col < p.N) p.P[(static_cast<int64_t>(g) * p.Ma + r) * p.N + col] = I;
                }
                const float t1 = static_cast<float>(I) * ws;
                acc[c][i] = acc[c][i] + t1 * s_as[g * R + r];
            }
            Pm[c] = v4i{0, 0, 0, 0};
        }
    };

    const int nsteps = (p.KT + 1) / 2;
    uint4 ga[P];
#pragma unroll
    for (int i = 0; i < P; ++i) ga[i] = load_a(i);
#pragma unroll
    for (int s = 0; s < D; ++s) load_w(s, s);
    *reinterpret_cast<uint4*>(&ring[0][tid * 16]) = ga[0];
    ga[0] = load_a(P);
    __syncthreads();   // staged scales and step 0

    for (int s0 = 0; s0 < nsteps; s0 += P) {
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int s = s0 + i;
            if (s >= nsteps) break;
            const uint8_t* slot = ring[i & 1];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int t = 2 * s + u;
                if (t >= p.KT) break;
                const int ws_slot = (2 * i + u) % D;
                v4i bw[CPW][2];
#pragma unroll
                for (int c = 0; c < CPW; ++c) {
                    const uint4 w = wb[ws_slot][c];
                    bw[c][0] = v4i{unpack_lo4(w.x), unpack_hi4(w.x), unpack_lo4(w.y), unpack_hi4(w.y)};
                    bw[c][1] = v4i{unpack_lo4(w.z), unpack_hi4(w.z), unpack_lo4(w.w), unpack_hi4(w.w)};
                }
                const uint4 h = *reinterpret_cast<const uint4*>(slot + u * 2048 + colq * 64 + q * 16);
                const uint4 l = *reinterpret_cast<const uint4*>(slot + u * 2048 + 1024 + colq * 64 + q * 16);
                int e[4], o[4];
                act_pair(h.x, l.x, e[0], o[0]);
                act_pair(h.y, l.y, e[1], o[1]);
                act_pair(h.z, l.z, e[2], o[2]);
                act_pair(h.w, l.w, e[3], o[3]);
                const v4i av0 = v4i{e[0], o[0], e[1], o[1]};
                const v4i av1 = v4i{e[2], o[2], e[3], o[3]};
                load_w(ws_slot, t + D);
#pragma unroll
                for (int c = 0; c < CPW; ++c) Pm[c] = mfma16(av0, bw[c][0], Pm[c]);
#pragma unroll
                for (int c = 0; c < CPW; ++c) Pm[c] = mfma16(av1, bw[c][1], Pm[c]);
                if ((t + 1) % p.tpg == 0 || t == p.KT - 1) fold(t / p.tpg);
            }
            // step s + 1 into the other slot (read last in step s - 1, which
            // every wave finished before the previous barrier)
            *reinterpret_cast<uint4*>(&ring[(i + 1) & 1][tid * 16]) = ga[(i + 1) % P];
            ga[(i + 1) % P] = load_a(s + 1 + P);
            __syncthreads();
        }
    }

#pragma unroll
    for (int c = 0; c < CPW; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = rowq + i, col = (nbw + wave * CPW + c) * 16 + colq;
            if (row < p.Ma && col < p.N)
                p.Y[static_cast<int64_t>(row) * p.ldy + col] = static_cast<uint16_t>(f32_to_bf16_bits(acc[c][i]));
        }
}

// Variants (rows x columns per workgroup, load depth, most waves):
//   Ma <= 16       16 x 32, depth 4, up to 12 waves (decode)
//   Ma <= 64       64 x 32, depth 2, up to 8 waves
//   Ma >  64       64 x 64, depth 2, up to 4 waves (prefill): twice the
//                  columns per activation read; one wave per SIMD
// Depth 2 at 64 rows keeps the operand ring within the register budget (at
// depth 4 the 64 x 32 tile spilled about 60 registers to scratch).
constexpr int mid_depth(int mt) { return mt == 1 ? 4 : 2; }
constexpr int kwmax_mid(int mt, int cpw) { return mt == 1 ? 12 : cpw > 2 ? 4 : 8; }

template <int MT, int CPW, bool ASYM, bool DUMP>
hipError_t launch_mid(const MidParams& p0, int kw, hipStream_t stream) {
    constexpr int D = mid_depth(MT), KWM = kwmax_mid(MT, CPW);
    MidParams p = p0;
    p.isum = false;
    p.gchunk = p.NG;
    // dynamic LDS: the staged scales, then the int32 group sums of as many
    // groups as fit (a slice each) and, past one chunk, the running fold
    const size_t staged = static_cast<size_t>(p.NG) * (2 * 16 * MT + 2 * 16 * CPW) * sizeof(float);
    const size_t slice = static_cast<size_t>(16 * MT) * 16 * CPW * sizeof(float);
    const dim3 grid(static_cast<unsigned>((p.NB + CPW - 1) / CPW), static_cast<unsigned>((p.Ma + 16 * MT - 1) / (16 * MT)));
    const int64_t wgs = static_cast<int64_t>(grid.x) * grid.y;
    // more than the default 64 KiB of dynamic LDS: the attribute, set once
    auto allow_lds = [](size_t lds) -> hipError_t {
        if (lds <= kMidLdsLimit) return hipSuccess;
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&gemm_midgroup_kernel<MT, CPW, KWM, D, ASYM, DUMP>),
            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kMidLdsIsum));
        return attr;
    };
    if (staged + slice > kMidLdsIsum) return hipErrorInvalidValue;
    // Waves per workgroup.  Few workgroups: K split at tile granularity
    // (about four tiles a wave) except on 9-16-row tiles, where whole groups
    // per wave are faster (MI355X, qkv / o us, tiles against groups: 1 row
    // 8.8 / 8.5 against 9.7 / 9.5, 16 rows 11.9 / 11.6 against 11.4 / 11.1, 64
    // rows 21.5 / 20.8 against 22.5 / 21.9); many workgroups: the caller's
    // count (one from 512 column pairs), at most two on prefill tiles.
    int w;
    if (wgs < 512) {
        w = MT == 1 && p.Ma > 8 ? std::min(p.NG, (p.NG + 1) / 2) : std::max(1, (p.KT + 3) / 4);
        if (CPW > 2) w = std::min(w, wgs >= 256 ? 2 : 4);
    } else {
        w = std::min(kw, p.NG);
        if (CPW > 2) w = std::min(w, wgs >= 1024 ? 1 : 2);
    }
    w = std::max(1, std::min(KWM, w));
    if (w > 1) {
        // Every wave adds its exact int32 group sums into LDS, after which the
        // workgroup folds the groups once in order -- the reference's fp32
        // order, bit for bit, whatever the split (the fp32 sums of whole-group
        // waves, added across waves, had put outputs outside 1 bf16 ulp of the
        // float64 value).  Groups whose sums do not fit at once go in chunks,
        // each output's fold carried between them.
        const size_t room = kMidLdsIsum - staged;
        int gch = static_cast<int>(std::min<size_t>(p.NG, room / slice));
        if (gch < p.NG) gch = static_cast<int>((room - slice) / slice);
        if (gch >= 1) {
            p.isum = true;
            p.gchunk = gch;
            const size_t lds = staged + static_cast<size_t>(gch + (gch < p.NG ? 1 : 0)) * slice;
            if (const hipError_t e = allow_lds(lds); e != hipSuccess) return e;
            gemm_midgroup_kernel<MT, CPW, KWM, D, ASYM, DUMP><<<grid, dim3(64 * w), lds, stream>>>(p);
            return hipGetLastError();
        }
    }
    // one wave walks every group in order
    if (const hipError_t e = allow_lds(staged); e != hipSuccess) return e;
    gemm_midgroup_kernel<MT, CPW, KWM, D, ASYM, DUMP><<<grid, dim3(64), staged, stream>>>(p);
    return hipGetLastError();
}

// The prefill variant's staged scales need twice the column slots; shapes
// whose group count leaves no room for them take the 64 x 32 variant.
bool mid_wide_fits(const MidParams& p) {
    return static_cast<size_t>(p.NG) * (2 * 64 + 2 * 64) * sizeof(float) + 64 * 64 * sizeof(float) <= kMidLdsLimit;
}

// Shapes for the shared-activation decode kernel: up to 16 rows on N wide
// enough that the per-wave plan walks K in one wave (>= 512 workgroups of two
// column blocks), with the staged scales within 56 KiB.
bool mid_shared_fits(const MidParams& p) {
    return p.Ma <= 16 && (p.NB + 1) / 2 >= 512 &&
           static_cast<size_t>(p.NG) * (2 * 16 + 2 * 16 * kShCPW * kShWaves) * sizeof(float) <= 56 * 1024;
}

template <bool ASYM, bool DUMP>
hipError_t launch_shared(const MidParams& p, hipStream_t stream) {
    const size_t lds = static_cast<size_t>(p.NG) * (2 * 16 + 2 * 16 * kShCPW * kShWaves) * sizeof(float);
    const dim3 grid(static_cast<unsigned>((p.NB + kShWaves * kShCPW - 1) / (kShWaves * kShCPW)));
    gemm_midgroup_shared_kernel<ASYM, DUMP><<<grid, dim3(64 * kShWaves), lds, stream>>>(p);
    return hipGetLastError();
}

// The staged values of an MT x 2 tile (16 MT rows, 32 columns) and one
// wave's fp32 sums within the LDS a launch can get.
bool mid_staged_fits(int64_t ng, int mt) {
    return static_cast<size_t>(ng) * (2 * 16 * mt + 2 * 32) * sizeof(float) + 16 * mt * 32 * sizeof(float) <=
           kMidLdsIsum;
}

// The int32 group sums of an MT x CPW tile fit the LDS beside the staged scales.
bool mid_isum_fits(const MidParams& p, int mt, int cpw) {
    return static_cast<size_t>(p.NG) * (2 * 16 * mt + 2 * 16 * cpw + 16 * mt * 16 * cpw) * sizeof(float) <= kMidLdsIsum;
}

template <bool ASYM, bool DUMP>
hipError_t launch_mt(const MidParams& p, int kw, hipStream_t stream) {
    if (mid_shared_fits(p)) return launch_shared<ASYM, DUMP>(p, stream);
    if (p.Ma <= 16) return launch_mid<1, 2, ASYM, DUMP>(p, kw, stream);
    if (p.Ma <= 64 || !mid_wide_fits(p)) {
        // 64-row tiles whose group sums exceed the LDS (many groups: down_proj's
        // 27 at group 1024) take 32-row tiles, whose sums fit, where the K
        // split over waves applies (few workgroups): the exact fold order at
        // the cost of reading the weights once per 32 rows
        const int64_t nb2 = (p.NB + 1) / 2;
        if (!mid_isum_fits(p, 4, 2) && mid_isum_fits(p, 2, 2) && nb2 * ((p.Ma + 31) / 32) < 512)
            return launch_mid<2, 2, ASYM, DUMP>(p, kw, stream);
        // more groups than 64 rows' staged values leave room for: 16-row tiles
        if (!mid_staged_fits(p.NG, 4)) return launch_mid<1, 2, ASYM, DUMP>(p, kw, stream);
        return launch_mid<4, 2, ASYM, DUMP>(p, kw, stream);
    }
    return launch_mid<4, 4, ASYM, DUMP>(p, kw, stream);
}

// w_q [N, kpad/2] as stored -> the tile layout (one thread per 16 bytes of a
// tile; columns past N and bytes past kpad/2 -- a last tile's padding half --
// are zero).
__global__ __launch_bounds__(256) void mid_tile_kernel(const uint8_t* __restrict__ wq, uint4* __restrict__ out, int64_t N,
                                                      int64_t kb, int64_t KT, int64_t chunks) {
    const int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (o >= chunks) return;
    const int64_t tile = o >> 6;
    const int l = static_cast<int>(o & 63);
    const int64_t nb = tile / KT, kt = tile - nb * KT;
    const int64_t col = nb * 16 + (l & 15);
    const int64_t b = kt * 64 + 16 * (l >> 4);
    out[o] = (col < N && b < kb) ? *reinterpret_cast<const uint4*>(wq + col * kb + b) : make_uint4(0u, 0u, 0u, 0u);
}

}  // namespace

int64_t midgroup_tiles_bytes(int64_t N, int64_t K, int64_t group) {
    return geom::col_blocks(N) * geom::k_tiles(K, group) * 1024;
}

hipError_t launch_midgroup_tile(const void* w_q, void* w_tiles, int64_t N, int64_t K, int64_t group,
                                hipStream_t stream) {
    const int64_t chunks = midgroup_tiles_bytes(N, K, group) / 16;
    if (chunks > 0)
        mid_tile_kernel<<<dim3(static_cast<unsigned>((chunks + 255) / 256)), dim3(256), 0, stream>>>(
            static_cast<const uint8_t*>(w_q), static_cast<uint4*>(w_tiles), N, geom::kpad(K, group) / 2,
            geom::k_tiles(K, group), chunks);
    return hipGetLastError();
}

int64_t midgroup_lds_bytes(int64_t Ma, int64_t K, int64_t group) {
    const int64_t ng = geom::num_groups(K, group);
    const int64_t mt = Ma <= 16 || !mid_staged_fits(ng, 4) ? 1 : 4;
    return (ng * (2 * 16 * mt + 2 * 32) + 16 * mt * 32) * 4;
}

int64_t midgroup_lds_max() { return static_cast<int64_t>(kMidLdsIsum); }

hipError_t launch_gemm_midgroup(const MidgroupArgs& a, hipStream_t stream) {
    MidParams p{};
    p.a_hi = static_cast<const uint8_t*>(a.a_hi);
    p.a_lo = static_cast<const uint8_t*>(a.a_lo);
    p.a_scale = static_cast<const uint16_t*>(a.a_scale);
    p.a_ksum = static_cast<const int32_t*>(a.a_ksum);
    p.w_q = static_cast<const uint8_t*>(a.w_q);
    p.w_scale = static_cast<const uint16_t*>(a.w_scale);
    p.w_zero = static_cast<const uint16_t*>(a.w_zero);
    p.Y = static_cast<uint16_t*>(a.y);
    p.P = static_cast<int32_t*>(a.partials);
    p.ldy = a.ldy;
    p.Ma = static_cast<int>(a.Ma);
    p.ld_as = static_cast<int>(a.ld_as);
    p.N = static_cast<int>(a.N);
    p.K = static_cast<int>(a.K);
    p.kpad = static_cast<int>(geom::kpad(a.K, a.group));
    p.kb = p.kpad / 2;
    p.KT = static_cast<int>(geom::ceil_div(p.kpad, 128));
    p.NG = static_cast<int>(geom::num_groups(a.K, a.group));
    p.NB = static_cast<int>(geom::col_blocks(a.N));
    p.tpg = static_cast<int>(geom::group_stride(a.group) / 128);
    p.a_bytes = static_cast<uint32_t>(a.Ma * static_cast<int64_t>(p.kb));
    p.wtiles = a.w_tiles;
    p.w_bytes = static_cast<uint32_t>(a.w_tiles ? midgroup_tiles_bytes(a.N, a.K, a.group)
                                                : a.N * static_cast<int64_t>(p.kb));
    // waves per workgroup: about two groups each, more for few column blocks
    const int64_t wgs = (p.NB + 1) / 2;
    const int kw = wgs >= 512 ? 1 : std::max(1, std::min(p.NG, static_cast<int>((p.NG + 1) / 2)));
    const bool asym = a.w_zero != nullptr, dump = a.partials != nullptr;
    if (asym) return dump ? launch_mt<true, true>(p, kw, stream) : launch_mt<true, false>(p, kw, stream);
    return dump ? launch_mt<false, true>(p, kw, stream) : launch_mt<false, false>(p, kw, stream);
}

}  // namespace w4a8
