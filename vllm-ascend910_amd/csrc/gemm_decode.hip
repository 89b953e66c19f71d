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
// activations (L2-resident), held D tiles ahead in a register ring.  All loads
// are raw buffer loads (SGPR descriptor + 32-bit offset) and unconditional:
// rows past M and tiles past the wave's range are addressed beyond the buffer
// ends and read as zero, so nothing is masked
// and the compiler can count loads in flight exactly.  Per 64-K slab each wave
// issues MT*CPW v_mfma_i32_16x16x64_i8; at each group end the int32
// accumulators fold into fp32 (acc += float(16*P) * w_scale).  The KW partial
// sums are reduced through LDS in a fixed order, and the token scale and the
// 1/16 of the nibble unpack are applied once at the end.  No workspace, no
// inter-workgroup communication (an agent-scope release/acquire pair costs
// about 10 us per call on MI355X, more than a K split across workgroups
// gains), deterministic results.
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
    int up_nb;         // SWIGLU: column blocks per half (gate block b pairs with up block b + up_nb)
    int nslab;         // 64-K slabs of the padded K axis (kpad / 64)
    int spg;           // 64-K slabs per group stride (ceil_to(group, 64) / 64)
    int gshift;        // GM 1: log2(tiles per group)
    int unit;          // tiles per K-split unit (group and tile aligned)
    int units;         // ceil(KT / unit)
    int cgroups;       // column groups (workgroups per row group)
    int rgroups;       // row groups of 16 * MT rows
    uint32_t a_bytes, w_bytes, s_bytes;
    // Fused activation quant (QM > 0): bf16 rows X [M, ldx] are quantised per
    // token inside the kernel into LDS (row stride lrs bytes); the workgroup of
    // column group 0 also writes a_q [M, lda_out] and a_scale [M].
    const uint16_t* X;
    int64_t ldx;
    int8_t* aq_out;
    int64_t lda_out;
    uint16_t* as_out;
    int lrs;
    int qcpr;          // 16-byte X chunks per row per lane (<= 8 / QM)
};

// Offset that every buffer here treats as out of range (reads return zero).
constexpr uint32_t kOOB = 0x80000000u;

// K is walked in the padded group layout (kgeom.h): group g occupies slabs
// [g*spg, (g+1)*spg) and only the last group may be shorter; the last slab
// nslab-1 always ends a group, and a last tile may hold a padding slab.
// GM: 0 = group stride 64 (a group per slab), 3 = stride 128 (a group per
// tile), 1 = stride 128 * 2^gshift, gshift >= 1 (groups end on a tile's upper
// slab, or on the last tile), 2 = any other stride (a group ends on either
// slab; a short last group may end right after another group in the same
// tile, so each slab carries its own scale), 4 = one group over all of K
// (per-channel scales): the K split then falls on any tile, the waves' int32
// sums are added exactly in LDS and folded once.  Modes 0 and 3 start every
// group with a zero accumulator operand; 1 and 2, whose group starts are
// runtime values, clear the accumulators after each fold.
// SWIGLU: the workgroup's first CPW/2 column blocks are gate blocks and the
// rest the matching up blocks (output column n = silu(y[:, n]) * y[:, n + N/2]);
// every column accumulates exactly as in the plain GEMM.
// QM > 0: the activation quant is fused (M <= QM <= 4, MT = 1, unpadded K;
// the launcher builds QM = 1 only):
// each wave loads the bf16 rows of its own K range, the waves' absmax meet in
// LDS, and each wave quantises its range into an LDS copy of A (the per-token
// arithmetic of quant_act.hip) that its MFMAs then read; the row loads are
// issued ahead of the weight ring, which streams meanwhile.
template <int MT, int CPW, int KWMAX, int D, int GM, bool SBF16, bool DUMP, bool SWIGLU, int QM>
__device__ __forceinline__ void decode_body(const DecodeParams& p) {
    static_assert(!SWIGLU || (CPW % 2 == 0 && !DUMP), "SwiGLU pairs column blocks and dumps nothing");
    static_assert(QM == 0 || (MT == 1 && QM <= 4 && !DUMP && !SWIGLU), "the fused quant serves at most 4 rows");
    constexpr int R = 16 * MT;
    constexpr int C = 16 * CPW;
    constexpr bool QF = QM > 0;
    // kw * R * C floats of reduction, sized at launch for the waves launched;
    // with QF followed by the quantised rows, a 64-byte zero block, the
    // waves' absmax and the rows' scale bits.
    extern __shared__ float red[];

    const int lane = threadIdx.x & 63;
    // Wave-uniform by construction; readfirstlane tells the compiler so, which
    // keeps the tile loop and fold conditions scalar.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kw = blockDim.x >> 6;
    constexpr int CG = SWIGLU ? CPW / 2 : CPW;   // column blocks per output group
    // Workgroup -> (column group, row group).  With several row groups the
    // ones that share a column group get consecutive ids of one XCD (ids are
    // dispatched round-robin over the 8 XCDs), so they run together and read
    // the weights through the same L2; ids past the column groups exit.
    int cgi = static_cast<int>(blockIdx.x), rgi = 0;
    if (p.rgroups > 1) {
        const int i = static_cast<int>(blockIdx.x) >> 3;
        const int j = i / p.rgroups;
        cgi = (j << 3) + static_cast<int>(blockIdx.x & 7);
        rgi = i - j * p.rgroups;
        if (cgi >= p.cgroups) return;
    }
    const int nb0 = cgi * CG;
    auto block_of = [&](int c) { return (SWIGLU && c >= CG) ? nb0 + (c - CG) + p.up_nb : nb0 + c; };
    const int rowq = 4 * (lane >> 4);  // first output row of this lane in a 16-row tile
    const int colq = lane & 15;        // A row / output column of this lane in a 16-block
    // Rows [m0, m0 + R) of the activations (more than R rows are split over
    // row groups that share the column blocks).
    const int m0 = rgi * R;
    // Token scales of this workgroup's rows: requested here, parked in LDS
    // just before the epilogue's barrier (a load issued in the epilogue would
    // add a memory round trip to the tail of every call).
    __shared__ uint32_t tsc[R];
    uint32_t ts_bits = 0;
    if constexpr (!QF) {
        if (static_cast<int>(threadIdx.x) < R && m0 + static_cast<int>(threadIdx.x) < p.M)
            ts_bits = p.a_scale[m0 + threadIdx.x];
    }

    // This wave's tile range [ta, tb).
    const int ua = (wave * p.units) / kw;
    const int ub = ((wave + 1) * p.units) / kw;
    const int ta = ua * p.unit;
    const int tb = min(p.KT, ub * p.unit);

    // Per-lane offsets are fixed for the whole K loop; the tile's uniform
    // offset goes into the descriptor base (make_rsrc_at).
    uint32_t wo[CPW], so[CPW], ao[MT][2];
    // QF: LDS regions (byte offsets from red) and this lane's A row address
    const int lq_a = kw * R * C * 4;
    const int lq_z = lq_a + QM * p.lrs;
    const int lq_m = lq_z + 64;
    const int lq_s = lq_m + kw * 16;
    char* const lds = reinterpret_cast<char*>(red);
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        // a column block past NB (odd NB, last workgroup) re-reads the last
        // block; its columns are past N and never stored
        const uint32_t nb = static_cast<uint32_t>(min(block_of(c), p.NB - 1));
        wo[c] = nb * static_cast<uint32_t>(p.KT) * 1024u + lane * 16u;   // tile 0
        so[c] = (nb * static_cast<uint32_t>(p.NG) * 16u + colq) * 2u;     // group 0
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        // rows past M start past the buffer end; a slab past K meets zero weights
        const uint32_t row = static_cast<uint32_t>(m0 + mt * 16 + colq);
        const uint32_t o = row < static_cast<uint32_t>(p.M) ? row * static_cast<uint32_t>(p.lda) + (lane >> 4) * 16u : kOOB;
        ao[mt][0] = o;         // slab 0 of tile 0
        ao[mt][1] = o + 64u;   // slab 1 (kOOB + 64 stays out of range)
    }

    // gend(t, h): the group whose scale slab h of tile t folds with (GM 1:
    // the group ending in tile t), clamped for the scale load.
    auto gend = [&](int t, int h) -> int {
        int g;
        if constexpr (GM == 0) g = 2 * t + h;
        else if constexpr (GM == 3) g = t;
        else if constexpr (GM == 1) g = t >> p.gshift;
        else g = (2 * t + h) / p.spg;
        return min(g, p.NG - 1);
    };

    // Register rings: D tiles of weights and of the scales of the groups
    // ending in them (two per tile for group 64, one otherwise), and DA tiles
    // of activations (L2-resident, so a shallower ring keeps the registers of
    // the 32- to 64-row tiles in budget).
    constexpr int NS = (GM == 1 || GM == 3 || GM == 4) ? 1 : 2;
    constexpr bool ONE = GM == 4;   // one group: int32 sums across the whole K range
    constexpr int DA = MT >= 3 ? 2 : D;
    static_assert(D % DA == 0, "activation ring depth must divide D");
    uint4 wb[D][CPW];
    uint4 ab[DA][MT][2];
    uint32_t sb[D][CPW][NS];
    auto load_a = [&](int sa, int t) {
        if constexpr (QF) {
            // rows past M read the zero block; tiles past the range re-read
            // the range's last tile (their weights are zero)
            const int tt = min(t, tb - 1);
            const bool real = colq < p.M;
            const char* base = lds + (real ? lq_a + colq * p.lrs + tt * 128 : lq_z) + (lane >> 4) * 16;
#pragma unroll
            for (int h = 0; h < 2; ++h) ab[sa][0][h] = *reinterpret_cast<const uint4*>(base + (real ? h * 64 : 0));
        } else {
            const auto ra = make_rsrc_at(p.A, static_cast<uint32_t>(min(t, p.KT - 1)) * 128u, p.a_bytes);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int h = 0; h < 2; ++h) ab[sa][mt][h] = buf_load16(ra, ao[mt][h]);
        }
    };
    auto load_slot = [&](int s, int t) {
        // tiles past this wave's range read zero weights (an empty descriptor)
        const auto rw = make_rsrc_at(p.W, static_cast<uint32_t>(t) * 1024u, t < tb ? p.w_bytes : 0u);
#pragma unroll
        for (int c = 0; c < CPW; ++c) wb[s][c] = buf_load16_nt(rw, wo[c]);
        if constexpr (ONE) return;   // the one scale per column is loaded once, before the loop
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            const auto rs = make_rsrc_at(p.S, static_cast<uint32_t>(gend(min(t, p.KT - 1), j)) * 32u, p.s_bytes);
#pragma unroll
            for (int c = 0; c < CPW; ++c) sb[s][c][j] = buf_load_u16(rs, so[c]);
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

    // `own`: the group lies in this wave's range (folds in the zero tiles past
    // the range add nothing and must not overwrite another wave's partials).
    auto fold = [&](int g, bool own, const uint32_t (&sc)[CPW][NS], int j) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
            const float ws = scale_to_f32<SBF16>(sc[c][j]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                if constexpr (DUMP) {
                    const int col = block_of(c) * 16 + colq;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int row = m0 + mt * 16 + rowq + i;
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

    // One pass over the D ring slots; PREFETCH refills each weight slot with
    // the tile D ahead (the last pass is peeled without it, so no weights past
    // the range are requested).  The activation ring is refilled DA ahead in
    // every pass.  Tiles of the last pass past tb hold zero weights: their
    // MFMAs add nothing and a fold there adds zero.
    auto pass = [&](int it, auto prefetch) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const int t = ta + it * D + s;
            uint32_t sc[CPW][NS];
#pragma unroll
            for (int c = 0; c < CPW; ++c)
#pragma unroll
                for (int j = 0; j < NS; ++j) sc[c][j] = sb[s][c][j];
            // Unpack the weight slot, then refill it; the activation slot is
            // used in place and refilled after its last MFMA (no copies).
            v4i b[CPW][2];
#pragma unroll
            for (int c = 0; c < CPW; ++c) unpack_tile_lane(wb[s][c], b[c][0], b[c][1]);
            if constexpr (decltype(prefetch)::value) load_slot(s, t + D);
            const auto& av = ab[s % DA];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const bool fresh = GM == 0 || (GM == 3 && h == 0);   // a group starts on this slab
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const uint4 v = av[mt][h];
                    const v4i a = {static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
#pragma unroll
                    for (int c = 0; c < CPW; ++c) P[mt][c] = mfma16(a, b[c][h], fresh ? v4i{0, 0, 0, 0} : P[mt][c]);
                }
                if (h == 1) load_a(s % DA, t + DA);
                if constexpr (ONE) {
                    // folded once, after the waves' sums meet
                } else if constexpr (GM == 0) {
                    // a padding slab past S folds group NG: zero partials,
                    // not dumped
                    fold(2 * t + h, t < tb, sc, h);
                } else if constexpr (GM == 3) {
                    if (h == 1) fold(t, t < tb, sc, 0);
                } else if constexpr (GM == 1) {
                    if (h == 1 && (((t + 1) & ((1 << p.gshift) - 1)) == 0 || t == p.KT - 1))
                        fold(t >> p.gshift, t < tb, sc, 0);
                } else {
                    const int sg = 2 * t + h;
                    if (sg < p.nslab && (((sg + 1) % p.spg) == 0 || sg == p.nslab - 1)) fold(sg / p.spg, t < tb, sc, h);
                }
            }
        }
    };

    const bool busy = tb > ta;
    // QF: this wave's real K range [k0, k1) of X in 16-byte chunks
    // c = lane + 64 i, loaded ahead of the weight ring (loads return in
    // order, so the quant below waits for X only).
    constexpr int QI = QF ? 8 / QM : 1;
    constexpr int QR = QF ? QM : 1;
    const int k0 = ta * 128, k1 = min(tb * 128, p.K);
    const int nch = max(0, (k1 - k0) >> 3);
    uint4 xv[QR][QI];
    if constexpr (QF) {
#pragma unroll
        for (int m = 0; m < QM; ++m)
#pragma unroll
            for (int i = 0; i < QI; ++i) {
                const int c = lane + 64 * i;
                const bool ok = m < p.M && i < p.qcpr && c < nch;
                xv[m][i] = ok ? *reinterpret_cast<const uint4*>(p.X + m * p.ldx + k0 + 8 * c) : make_uint4(0u, 0u, 0u, 0u);
            }
    }
    uint32_t ws1[CPW];   // ONE: the scale of each column block's columns of this lane
    if (busy) {
#pragma unroll
        for (int s = 0; s < D; ++s) load_slot(s, ta + s);
    }
    if constexpr (ONE) {
        const auto rs = make_rsrc(p.S, p.s_bytes);
#pragma unroll
        for (int c = 0; c < CPW; ++c) ws1[c] = buf_load_u16(rs, so[c]);
    }
    if constexpr (QF) {
        uint32_t am[QM];
#pragma unroll
        for (int m = 0; m < QM; ++m) {
            am[m] = 0u;
#pragma unroll
            for (int i = 0; i < QI; ++i) am[m] = max(am[m], abs_bits_max8(xv[m][i]));
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1)
                am[m] = max(am[m], static_cast<uint32_t>(__shfl_xor(static_cast<int>(am[m]), off, 64)));
        }
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < QM; ++m) reinterpret_cast<uint32_t*>(lds + lq_m)[wave * 4 + m] = am[m];
        }
        if (wave == 0 && lane < 16) reinterpret_cast<uint32_t*>(lds + lq_z)[lane] = 0u;
        __syncthreads();
        const bool writer = cgi == 0 && rgi == 0;   // one workgroup emits a_q / a_scale
#pragma unroll
        for (int m = 0; m < QM; ++m) {
            if (m >= p.M) break;
            // lane w < kw reads wave w's absmax, then a wave-wide max
            uint32_t amax = lane < kw ? reinterpret_cast<const uint32_t*>(lds + lq_m)[lane * 4 + m] : 0u;
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1)
                amax = max(amax, static_cast<uint32_t>(__shfl_xor(static_cast<int>(amax), off, 64)));
            amax = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(amax)));
            const uint32_t sbits = scale_from_amax(amax);
            if (wave == 0 && lane == 0) {
                reinterpret_cast<uint32_t*>(lds + lq_s)[m] = sbits;
                if (writer) p.as_out[m] = static_cast<uint16_t>(sbits);
            }
            const RowScale q = row_scale(bf16_bits_to_f32(sbits));
            auto emit = [&](auto fast) __attribute__((always_inline)) {
                constexpr bool F = decltype(fast)::value;
#pragma unroll
                for (int i = 0; i < QI; ++i) {
                    const int c = lane + 64 * i;
                    if (i < p.qcpr && c < nch) {
                        const uint4 v = xv[m][i];
                        uint2 o;
                        o.x = quant2<F>(v.x, q) | (quant2<F>(v.y, q) << 16);
                        o.y = quant2<F>(v.z, q) | (quant2<F>(v.w, q) << 16);
                        *reinterpret_cast<uint2*>(lds + lq_a + m * p.lrs + k0 + 8 * c) = o;
                        if (writer) *reinterpret_cast<uint2*>(p.aq_out + m * p.lda_out + k0 + 8 * c) = o;
                    }
                }
            };
            if (q.fast) emit(std::true_type{});
            else emit(std::false_type{});
        }
    }
    if (busy) {
#pragma unroll
        for (int s = 0; s < DA; ++s) load_a(s, ta + s);
        const int iters = (tb - ta + D - 1) / D;
        for (int it = 0; it + 1 < iters; ++it) pass(it, std::true_type{});
        pass(iters - 1, std::false_type{});
    }

    // Fixed-order reduction of the kw wave partials, then the epilogue.  With
    // one group the waves' int32 sums are added (exactly, so the order does
    // not matter) and folded with the column's scale once.
    __shared__ float wsl[ONE ? C : 1];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int c = 0; c < CPW; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float* r = &red[wave * R * C + (mt * 16 + rowq + i) * C + c * 16 + colq];
                if constexpr (ONE) *reinterpret_cast<int*>(r) = P[mt][c][i];
                else *r = acc[mt][c][i];
            }
    if constexpr (ONE) {
        if (wave == 0 && lane < 16) {
#pragma unroll
            for (int c = 0; c < CPW; ++c) wsl[c * 16 + colq] = scale_to_f32<SBF16>(ws1[c]);
        }
    }
    if constexpr (!QF) {
        if (static_cast<int>(threadIdx.x) < R) tsc[threadIdx.x] = ts_bits;
    }
    __syncthreads();
    // the fp32 sum (before the token scale) of local element e = row * C + cc
    auto colsum = [&](int e, int cc) -> float {
        if constexpr (ONE) {
            int isum = reinterpret_cast<const int*>(red)[e];
            for (int w = 1; w < kw; ++w) isum += reinterpret_cast<const int*>(red)[w * R * C + e];
            if constexpr (DUMP) {
                const int row = e / C, col = block_of(cc / 16) * 16 + cc % 16;
                if (m0 + row < p.M && col < p.N) p.P[static_cast<int64_t>(m0 + row) * p.N + col] = isum >> 4;
            }
            return static_cast<float>(isum) * wsl[cc];
        } else {
            float sum = red[e];
            for (int w = 1; w < kw; ++w) sum += red[w * R * C + e];
            return sum;
        }
    };
    if constexpr (SWIGLU) {
        constexpr int CH = C / 2;
        for (int e = threadIdx.x; e < R * CH; e += blockDim.x) {
            const int row = e / CH;
            const int cc = e - row * CH;
            const int col = nb0 * 16 + cc;
            if (m0 + row >= p.M || col >= p.up_nb * 16) continue;
            const float sg = colsum(row * C + cc, cc), su = colsum(row * C + CH + cc, CH + cc);
            const float ts = bf16_bits_to_f32(tsc[row]) * 0.0625f;
            p.Y[static_cast<int64_t>(m0 + row) * p.ldy + col] = static_cast<uint16_t>(swiglu_bf16_bits(sg * ts, su * ts));
        }
    } else {
        for (int e = threadIdx.x; e < R * C; e += blockDim.x) {
            const int row = e / C;
            const int col = nb0 * 16 + (e - row * C);
            if (m0 + row >= p.M || col >= p.N) continue;
            const float sum = colsum(e, e - row * C);
            const uint32_t tsb = QF ? reinterpret_cast<const uint32_t*>(lds + lq_s)[row] : tsc[row];
            const float ts = bf16_bits_to_f32(tsb) * 0.0625f;
            p.Y[static_cast<int64_t>(m0 + row) * p.ldy + col] = static_cast<uint16_t>(f32_to_bf16_bits(sum * ts));
        }
    }
}

template <int MT, int CPW, int KWMAX, int D, int GM, bool SBF16, bool DUMP, bool SWIGLU>
__global__ __launch_bounds__(64 * KWMAX) void gemm_decode_kernel(const DecodeParams p) {
    decode_body<MT, CPW, KWMAX, D, GM, SBF16, DUMP, SWIGLU, 0>(p);
}

// The fused quant + GEMM of one row (its own name in kernel traces).
template <int KWMAX, int GM, bool SBF16>
__global__ __launch_bounds__(64 * KWMAX) void linear_decode_kernel(const DecodeParams p) {
    decode_body<1, 2, KWMAX, 4, GM, SBF16, false, false, 1>(p);
}

int gcd_i(int a, int b) {
    while (b) {
        const int t = a % b;
        a = b;
        b = t;
    }
    return a;
}

// Most waves per workgroup a variant is built for (its register budget: the
// 64-row, 4-block variant needs 256 VGPRs at 2 waves per SIMD).
constexpr int kwmax_for(int mt, int cpw, int d) {
    // one 16-row tile of one column block with a 4-deep ring fits 16 waves (128 VGPRs)
    return mt == 1 ? (cpw >= 4 ? 8 : (cpw == 1 && d <= 4 ? 16 : 12)) : (mt == 2 || cpw <= 2 ? 8 : 4);
}

// MODE: 0 = plain, 1 = plain with partial dump, 2 = SwiGLU epilogue.
template <int MT, int CPW, int D, int GM, int MODE>
hipError_t launch_g(const DecodeParams& p, int kw, bool sbf16, hipStream_t stream) {
    constexpr int KWM = kwmax_for(MT, CPW, D);
    constexpr bool DUMP = MODE == 1, SWIGLU = MODE == 2;
    if constexpr (SWIGLU && CPW % 2 != 0) {
        return hipErrorInvalidValue;
    } else {
        const int w = std::max(1, std::min(kw, KWM));
        constexpr int CG = SWIGLU ? CPW / 2 : CPW;
        const int nbg = SWIGLU ? p.up_nb : p.NB;
        DecodeParams q = p;
        q.cgroups = (nbg + CG - 1) / CG;
        q.rgroups = (p.M + 16 * MT - 1) / (16 * MT);
        const int64_t nwg = q.rgroups > 1 ? int64_t{8} * ((q.cgroups + 7) / 8) * q.rgroups : q.cgroups;
        const dim3 grid(static_cast<unsigned>(nwg)), block(64 * w);
        const size_t lds = static_cast<size_t>(w) * 16 * MT * 16 * CPW * sizeof(float);
        if (sbf16) gemm_decode_kernel<MT, CPW, KWM, D, GM, true, DUMP, SWIGLU><<<grid, block, lds, stream>>>(q);
        else gemm_decode_kernel<MT, CPW, KWM, D, GM, false, DUMP, SWIGLU><<<grid, block, lds, stream>>>(q);
        return hipGetLastError();
    }
}

// Group mode: one group over all of K -> 4; otherwise by group stride: 64 ->
// 0; 128 -> 3; 128 * 2^s, s >= 1 -> 1; anything else -> 2.
int group_mode(int spg, int ng) {
    if (ng == 1) return 4;
    if (spg == 1) return 0;
    if (spg == 2) return 3;
    if (spg % 2 == 0 && ((spg / 2) & (spg / 2 - 1)) == 0) return 1;
    return 2;
}

template <int MT, int CPW, int D, int MODE>
hipError_t launch_v(const DecodeParams& p, int kw, bool sbf16, hipStream_t stream) {
    switch (group_mode(p.spg, p.NG)) {
        case 0: return launch_g<MT, CPW, D, 0, MODE>(p, kw, sbf16, stream);
        case 1: return launch_g<MT, CPW, D, 1, MODE>(p, kw, sbf16, stream);
        case 3: return launch_g<MT, CPW, D, 3, MODE>(p, kw, sbf16, stream);
        case 4: return launch_g<MT, CPW, D, 4, MODE>(p, kw, sbf16, stream);
        default: return launch_g<MT, CPW, D, 2, MODE>(p, kw, sbf16, stream);
    }
}

// The variants that are built: (MT, D, CPW); the SwiGLU epilogue needs an
// even CPW.
template <int MODE>
hipError_t dispatch(const DecodeParams& p, const DecodeConfig& c, bool sbf16, hipStream_t s) {
    // c.MT > 0: workgroups of 16 * c.MT rows, gridDim.y of them
    const int mt = c.MT > 0 ? std::min(c.MT, (p.M + 15) / 16) : (p.M + 15) / 16;
    if constexpr (MODE != 2) {
        if (mt == 1 && c.D == 8 && c.CPW == 1) return launch_v<1, 1, 8, MODE>(p, c.KW, sbf16, s);
        if (mt == 1 && c.D == 4 && c.CPW == 1) return launch_v<1, 1, 4, MODE>(p, c.KW, sbf16, s);
        if (mt == 2 && c.D == 4 && c.CPW == 1) return launch_v<2, 1, 4, MODE>(p, c.KW, sbf16, s);
    }
    if (mt == 1 && c.D == 4 && c.CPW == 2) return launch_v<1, 2, 4, MODE>(p, c.KW, sbf16, s);
    if (mt == 1 && c.D == 2 && c.CPW == 4) return launch_v<1, 4, 2, MODE>(p, c.KW, sbf16, s);
    if (mt == 2 && c.D == 4 && c.CPW == 2) return launch_v<2, 2, 4, MODE>(p, c.KW, sbf16, s);
    if (mt == 2 && c.D == 2 && c.CPW == 4) return launch_v<2, 4, 2, MODE>(p, c.KW, sbf16, s);
    if (mt == 3 && c.D == 4 && c.CPW == 2) return launch_v<3, 2, 4, MODE>(p, c.KW, sbf16, s);
    if (mt == 4 && c.D == 4 && c.CPW == 2) return launch_v<4, 2, 4, MODE>(p, c.KW, sbf16, s);
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
    p.up_nb = a.swiglu ? static_cast<int>(a.N / 2 / geom::kTileN) : 0;
    p.nslab = static_cast<int>(geom::kpad(a.K, a.group) / 64);
    p.spg = static_cast<int>(geom::group_stride(a.group) / 64);
    p.gshift = 0;
    while ((2 << p.gshift) < p.spg) ++p.gshift;
    // Rows end at kpad; reads past it (the padding slab of a last tile) meet
    // zero weights, and in the last row they are out of range (zero).
    p.a_bytes = static_cast<uint32_t>((a.M - 1) * a.lda + geom::kpad(a.K, a.group));
    p.w_bytes = static_cast<uint32_t>(p.NB * static_cast<int64_t>(p.KT) * geom::kTileBytes);
    p.s_bytes = static_cast<uint32_t>(p.NB * static_cast<int64_t>(p.NG) * 16 * 2);
    // K-split boundaries fall on both tile (2 slabs) and group boundaries --
    // any tile for a single group, whose int32 sums the waves add before the fold.
    p.unit = p.NG == 1 ? 1 : (2 * p.spg / gcd_i(2, p.spg)) / 2;
    p.units = (p.KT + p.unit - 1) / p.unit;
    return p;
}

// Fused quant + GEMM: MT = 1, CPW = 2, D = 4, plain epilogue, one row.
template <int GM, bool SBF16>
hipError_t launch_fused_g(const DecodeParams& p, int kw, size_t lds, hipStream_t stream) {
    constexpr int KWM = kwmax_for(1, 2, 4);
    linear_decode_kernel<KWM, GM, SBF16><<<dim3(static_cast<unsigned>(p.cgroups)), dim3(64 * kw), lds, stream>>>(p);
    return hipGetLastError();
}

hipError_t launch_fused(const DecodeParams& p, int kw, size_t lds, bool sbf16, hipStream_t s) {
    switch (group_mode(p.spg, p.NG)) {
        case 4: return sbf16 ? launch_fused_g<4, true>(p, kw, lds, s) : launch_fused_g<4, false>(p, kw, lds, s);
        case 0: return sbf16 ? launch_fused_g<0, true>(p, kw, lds, s) : launch_fused_g<0, false>(p, kw, lds, s);
        case 1: return sbf16 ? launch_fused_g<1, true>(p, kw, lds, s) : launch_fused_g<1, false>(p, kw, lds, s);
        case 3: return sbf16 ? launch_fused_g<3, true>(p, kw, lds, s) : launch_fused_g<3, false>(p, kw, lds, s);
        default: return sbf16 ? launch_fused_g<2, true>(p, kw, lds, s) : launch_fused_g<2, false>(p, kw, lds, s);
    }
}

// The fused plan for a problem, or false when the two-kernel path applies.
struct FusedPlan {
    DecodeParams p;
    int kw, qm;
    size_t lds;
};

bool plan_fused(const GemmArgs& a, const uint16_t* x, int64_t ldx, FusedPlan& f) {
    // One row only: each workgroup quantises the rows of its K range, so the
    // quant work is repeated per column group.  (Measured on MI355X: one row
    // saves 0.5-3 us per call over the quant kernel + GEMM pair on narrow N
    // and ~2 us on gate_up's 1728 column groups; at 2-4 rows the
    // per-workgroup quant costs more than the launch it saves.)
    if (a.M != 1 || a.swiglu || a.partials || !geom::is_unpadded(a.K, a.group)) return false;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || ldx % 8 != 0) return false;
    const DecodeConfig c = decode_config(a.M, a.N, a.K, a.group);
    if (c.D != 4 || c.CPW != 2 || c.MT != 0 || c.WIDE) return false;
    f.p = make_params(a);
    f.p.cgroups = (f.p.NB + 1) / 2;
    f.p.rgroups = 1;
    f.qm = 1;
    // The GEMM's own K split (same waves, same ranges, same reduction order),
    // so the fused call equals quant + GEMM bit for bit.
    f.kw = c.KW;
    if (f.kw < 1 || f.kw > kwmax_for(1, 2, 4)) return false;
    const int tiles = f.p.unit * ((f.p.units + f.kw - 1) / f.kw);   // most tiles a wave owns
    f.p.qcpr = (tiles + 3) / 4;                                     // 16-byte chunks per row per lane
    if (f.p.qcpr > 8 / f.qm) return false;
    f.p.lrs = f.p.KT * 128 + 16;   // 16-byte skew: the rows' reads fall on different banks
    f.lds = static_cast<size_t>(f.kw) * 16 * 32 * 4 + static_cast<size_t>(f.qm) * f.p.lrs + 64 + f.kw * 16 + 16;
    if (f.lds > 64 * 1024) return false;
    f.p.X = x;
    f.p.ldx = ldx;
    return true;
}

}  // namespace

bool linear_fusable(const GemmArgs& a, const uint16_t* x, int64_t ldx) {
    FusedPlan f;
    return plan_fused(a, x, ldx, f);
}

hipError_t launch_linear_fused(const GemmArgs& a, const uint16_t* x, int64_t ldx, int8_t* a_q, int64_t lda,
                               uint16_t* a_scale, hipStream_t stream) {
    FusedPlan f;
    if (!plan_fused(a, x, ldx, f)) return hipErrorInvalidValue;
    f.p.aq_out = a_q;
    f.p.lda_out = lda;
    f.p.as_out = a_scale;
    return launch_fused(f.p, f.kw, f.lds, a.scale_bf16, stream);
}

namespace {

// The decode kernel's own plans (no wide layout): every shape has one.
DecodeConfig rows_config(int64_t M, int64_t N, int64_t K, int64_t group) {
    const int mt = static_cast<int>((M + 15) / 16);
    const int KT = static_cast<int>(geom::k_tiles(K, group));
    const int64_t NB = geom::col_blocks(N);
    DecodeConfig c{4, 2, 4};
    const int64_t wgs = (NB + 1) / 2;
    if (wgs >= 4 * device_cu_count()) {
        // Wide N already gives >= 4 workgroups of all rows per CU: one wave each
        // -- two for a single row, whose fused-quant plan (the same split)
        // needs a wave's K range to fit its prologue's registers.
        if (mt == 1) c.KW = M == 1 ? 2 : 1;
        else c = DecodeConfig{4, 2, 1};
    } else if (mt == 1 || (mt == 2 && KT >= 128)) {
        // Split K so that each wave holds about one ring (4 tiles) of its
        // range -- but long K (>= 128 tiles) streams better with six longer
        // waves (four past 8 rows); a single row takes eight, which its fused
        // quant prologue prefers (down_proj linear 20.7 against 21.4 us at
        // seven; that plan uses the GEMM's split).
        const int cap = KT >= 128 ? (M == 1 ? 8 : (M <= 8 ? 6 : 4)) : 12;
        c.KW = std::max(1, std::min(cap, (KT + 3) / 4));
    } else {
        // More than 16 rows on narrow N with short K: row groups that share
        // each column group, four column blocks each, so every workgroup's
        // activation rows serve twice the columns of a two-block group (the
        // L2 reads of A bound these shapes: qkv M=64 17.5 -> 14.3 us).
        // 16-row groups (six waves up to 28 rows, four past) while they fit
        // the CUs in one round; past that 32-row groups of four waves, which
        // read each column group's weights half as often (qkv M=64 14.3 ->
        // 13.5 us, o M=64 14.1 -> 13.1 us; o M=48 stays at 10 us on 240
        // 16-row workgroups against 12.6 us).
        const int64_t cg = (NB + 3) / 4;
        if (cg * ((M + 15) / 16) <= device_cu_count()) c = DecodeConfig{2, 4, M <= 28 ? 6 : 4, 1};
        else c = DecodeConfig{2, 4, 4, 2};
    }
    return c;
}

}  // namespace

DecodeConfig decode_config(int64_t M, int64_t N, int64_t K, int64_t group) {
    // Picked from sweeps over ring depths, column blocks per workgroup, waves
    // per workgroup and K splits on MI355X at the QwQ-32B projection shapes.
    const int mt = static_cast<int>((M + 15) / 16);
    const int KT = static_cast<int>(geom::k_tiles(K, group));
    const int64_t NB = geom::col_blocks(N);
    const int64_t wgs = (NB + 1) / 2;
    DecodeConfig c{4, 2, 1};
    if (M > 8 && wgs >= 4 * device_cu_count()) {
        // Wide N past 8 rows: the activations each decode workgroup reads
        // weigh as much as its weights; four column waves share them in LDS.
        c.WIDE = mt == 1 ? kWide1x2 : (mt == 2 ? kWide2x2 : kWide4x2);
        return c;
    }
    if (M > 8 && KT >= 128) {
        // Narrow N, long K, past 8 rows: the same sharing with one column
        // block per wave, K split over workgroups (at least 8 tiles each):
        // ~3.75 per CU for the 16-row layout, ~2.5 for 32 rows, ~1.9 for 64
        // (the lighter the workgroup, the more of them; down_proj on 256
        // CUs: 960 / 640 / 480 workgroups, 12, 8 and 6 splits).
        c.WIDE = mt == 1 ? kWide1x1 : (mt == 2 ? kWide2x1 : kWide4x1);
        const int64_t cg = (NB + 3) / 4;
        const int64_t cus = device_cu_count();
        const int64_t target = mt == 1 ? cus * 15 / 4 : (mt == 2 ? cus * 5 / 2 : cus * 15 / 8);
        const int64_t s = std::min<int64_t>({(target + cg / 2) / cg, int64_t{16}, KT / 8});
        c.SPLITS = static_cast<int>(std::max<int64_t>(s, 1));
        return c;
    }
    return rows_config(M, N, K, group);
}

int64_t decode_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group) {
    const DecodeConfig c = decode_config(M, N, K, group);
    return c.WIDE && c.SPLITS > 1 ? wide_workspace_bytes(M, N, K, group, c.SPLITS) : 0;
}

hipError_t launch_gemm_decode_cfg(const GemmArgs& a, const DecodeConfig& cfg, hipStream_t stream) {
    if (cfg.WIDE) {
        if (!a.swiglu || wide_layout_pairs(cfg.WIDE)) return launch_gemm_wide(a, cfg.WIDE, cfg.SPLITS, stream);
        // the one-block layouts have no SwiGLU pairs: the decode kernel's plan
        return launch_gemm_decode_cfg(a, rows_config(a.M, a.N, a.K, a.group), stream);
    }
    const DecodeParams p = make_params(a);
    if (a.swiglu) return dispatch<2>(p, cfg, a.scale_bf16, stream);
    return a.partials ? dispatch<1>(p, cfg, a.scale_bf16, stream) : dispatch<0>(p, cfg, a.scale_bf16, stream);
}

hipError_t launch_gemm_decode(const GemmArgs& a, hipStream_t stream) {
    return launch_gemm_decode_cfg(a, decode_config(a.M, a.N, a.K, a.group), stream);
}

}  // namespace w4a8
