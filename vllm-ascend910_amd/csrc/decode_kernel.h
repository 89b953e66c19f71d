#pragma once
// Decode-shaped W4A8 GEMM (M <= 64): HBM weight-stream bound.  The kernel
// body, shared by gemm_decode.hip and gemm_decode_staged.hip (each builds its
// own variants).
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
namespace dec {

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

// Staged activations (SA > 0): a staged row's LDS stride (128 bytes plus a
// 16-byte skew that spreads the rows' reads over the banks), the groups whose
// scales one pass of D tiles can fold, and one wave's LDS area (a 16-byte
// dump slot and two pass buffers; at least the wave's reduction rows, which
// reuse it).
constexpr int kStRow = 144;
__host__ __device__ constexpr int st_pass_groups(int gm, int d) { return gm == 0 ? 2 * d : d; }
__host__ __device__ constexpr int st_wave_bytes(int m, int cpw, int gm, int d) {
    const int ssb = gm == 4 ? 0 : cpw * st_pass_groups(gm, d) * 32;
    const int v = 16 + 2 * (d * m * kStRow + ssb);
    return v > 16 * 16 * cpw * 4 ? v : 16 * 16 * cpw * 4;
}

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
// issued ahead of the weight ring, which streams meanwhile.  Its group scales
// are staged per pass as below.  QW > 0 (one row of at most 64 * 8 * QW
// elements): every wave reads the whole row instead (QW 16-byte chunks per
// lane, L2 hits after the first reads) and finds the absmax itself, so the
// prologue has no barrier and no wave waits for another's row slice; it
// quantises only its own range, and rows past M read row 0 (their outputs are
// never stored).  Measured on MI355X (cold weights, graph replays): qkv
// 8.36 -> 7.56 us, o_proj 7.78 -> 7.14 us, the same output bits.
// SA > 0: staged activations and scales (M <= 8, MT = 1, D = 4).  A 16-row
// tile of a few real rows wastes most of each per-tile activation load (the
// 16-byte lane loads of rows past M still occupy the load pipeline), and the
// scale loads move 32 bytes per instruction.  Instead each wave walks its
// range in passes of D tiles and, two passes ahead, fetches a pass's real
// rows (M * D * 128 bytes, SA 16-byte lane loads) and the scales of the
// groups that can end in it (one 16-byte lane load) into registers; at the
// start of the pass before, it writes them to one of two LDS buffers of its
// own, from which the ring reads each tile's activations (rows past M re-read
// row 0: their outputs are never stored) and each fold its scales.  Only the
// wave that owns a buffer touches it, and LDS operations of a wave complete in
// issue order, so no barrier is needed; the reduction reuses the same area
// once the wave's loop is over.
template <int MT, int CPW, int KWMAX, int D, int GM, bool SBF16, bool DUMP, bool SWIGLU, int QM, int SA = 0, int QW = 0>
__device__ __forceinline__ void decode_body(const DecodeParams& p) {
    static_assert(!SWIGLU || (CPW % 2 == 0 && !DUMP), "SwiGLU pairs column blocks and dumps nothing");
    static_assert(QM == 0 || (MT == 1 && QM <= 4 && !DUMP && !SWIGLU), "the fused quant serves at most 4 rows");
    static_assert(SA == 0 || (MT == 1 && QM == 0 && D == 4 && CPW <= 2), "staged activations: one row tile, 4-tile passes");
    constexpr int R = 16 * MT;
    constexpr int C = 16 * CPW;
    constexpr bool QF = QM > 0;
    constexpr bool ST = SA > 0;
    // kw * R * C floats of reduction, sized at launch for the waves launched;
    // with QF followed by the quantised rows, a 64-byte zero block, the
    // waves' absmax and the rows' scale bits.  ST: kw areas of st_wave_bytes
    // (a 16-byte dump slot for the staging lanes past the data, then two pass
    // buffers of st_ab activation bytes and SSB scale bytes); wave w's
    // reduction rows start at its own area.
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

    // graw(t, h): the group whose scale slab h of tile t folds with (GM 1:
    // the group ending in tile t); gend clamps it for the scale load.
    // gfirst(t): the group of tile t's first slab.
    auto graw = [&](int t, int h) -> int {
        if constexpr (GM == 0) return 2 * t + h;
        else if constexpr (GM == 3) return t;
        else if constexpr (GM == 1) return t >> p.gshift;
        else return (2 * t + h) / p.spg;
    };
    auto gend = [&](int t, int h) -> int { return min(graw(t, h), p.NG - 1); };
    auto gfirst = [&](int t) -> int {
        if constexpr (GM == 0) return 2 * t;
        else if constexpr (GM == 3) return t;
        else if constexpr (GM == 1) return t >> p.gshift;
        else return (2 * t) / p.spg;
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

    // STS: group scales staged per pass (with the activations for ST; the
    // fused quant, whose rows are in LDS already, stages the scales alone).
    // This wave's staging area (bytes from red): a 16-byte dump slot, then
    // pass buffers at +16 and +16 + st_buf, each st_ab bytes of rows (slot s,
    // row r at (s * M + r) * kStRow; ST only) and the scales of NGP groups per
    // column block (block c, group g0 + i at st_ab + (c * NGP + i) * 32).
    // ST areas start at wave * st_wave; QF areas follow the quant's regions.
    constexpr bool STS = ST || (QF && !ONE);
    constexpr int NGP = st_pass_groups(GM, D);
    const int st_ab = ST ? D * p.M * kStRow : 0;
    const int st_buf = st_ab + ((STS && !ONE) ? CPW * NGP * 32 : 0);
    const int st_wave = ST ? st_wave_bytes(p.M, CPW, GM, D) : R * C * 4;
    const int lw = ST ? wave * st_wave : lq_s + 16 + wave * (16 + 2 * st_buf);
    constexpr int SAN = ST ? SA : 1;
    // Per staged chunk i (lane + 64 i: row r = chunk / 32, 16-byte piece q =
    // chunk % 32 of the pass's 512 bytes per row): its offset in the pass's
    // rows and in a buffer, kOOB past the M rows (read as zero, written to the
    // dump slot).  The scale chunk of lane l < CPW * NGP * 2: block l / (2 NGP),
    // group g0 + (l / 2) % NGP, half l % 2.
    uint32_t sg[SAN], sl[SAN];
    uint32_t sgs = kOOB, sls = kOOB, arow = 0;
    const int sgi = (lane >> 1) % NGP;
    uint4 xs[SAN], xsc;
    if constexpr (STS) {
#pragma unroll
        for (int i = 0; i < SA; ++i) {
            const int c = lane + 64 * i, r = c >> 5, q = c & 31;
            const bool real = r < p.M;
            sg[i] = real ? static_cast<uint32_t>(r) * static_cast<uint32_t>(p.lda) + q * 16u : kOOB;
            sl[i] = real ? static_cast<uint32_t>(((q >> 3) * p.M + r) * kStRow + (q & 7) * 16) : kOOB;
        }
        if constexpr (!ONE) {
            if (lane < CPW * NGP * 2) {
                const uint32_t nb = static_cast<uint32_t>(min(block_of(lane / (2 * NGP)), p.NB - 1));
                sgs = (nb * static_cast<uint32_t>(p.NG) + sgi) * 32u + (lane & 1) * 16u;
                sls = static_cast<uint32_t>(st_ab + lane * 16);
            }
        }
        // rows past M read row 0 (their outputs are never stored)
        arow = static_cast<uint32_t>((colq < p.M ? colq : 0) * kStRow + (lane >> 4) * 16);
    }
    // Fetch pass pi's rows and scales into registers (a pass past the range
    // reads zeros through empty descriptors).
    auto stage_issue = [&](int pi) {
        const int t0 = ta + pi * D;
        const bool live = t0 < tb;
        if constexpr (ST) {
            const auto ra = make_rsrc_at(p.A, static_cast<uint32_t>(t0) * 128u, live ? p.a_bytes : 0u);
#pragma unroll
            for (int i = 0; i < SAN; ++i) xs[i] = buf_load16(ra, sg[i]);
        }
        if constexpr (!ONE) {
            const int g0 = gfirst(t0);
            const auto rs = make_rsrc_at(p.S, static_cast<uint32_t>(g0) * 32u, live ? p.s_bytes : 0u);
            xsc = buf_load16(rs, sgi < p.NG - g0 ? sgs : kOOB);
        }
    };
    // Write the fetched pass pi into its buffer.
    auto stage_commit = [&](int pi) {
        char* const buf = lds + lw + 16 + (pi & 1) * st_buf;
        if constexpr (ST) {
#pragma unroll
            for (int i = 0; i < SAN; ++i) *reinterpret_cast<uint4*>(sl[i] != kOOB ? buf + sl[i] : lds + lw) = xs[i];
        }
        if constexpr (!ONE) *reinterpret_cast<uint4*>(sls != kOOB ? buf + sls : lds + lw) = xsc;
    };
    // Activations of slot si of pass pi into ring slot sa.
    auto load_a_st = [&](int sa, int pi, int si) {
        const char* const base = lds + lw + 16 + (pi & 1) * st_buf + si * p.M * kStRow + arow;
        ab[sa][0][0] = *reinterpret_cast<const uint4*>(base);
        ab[sa][0][1] = *reinterpret_cast<const uint4*>(base + 64);
    };
    auto load_a = [&](int sa, int t) {
        if constexpr (QF) {
            // rows past M read the zero block; tiles past the range re-read
            // the range's last tile (their weights are zero)
            const int tt = min(t, tb - 1);
            const bool real = colq < p.M;
            if constexpr (QW > 0) {
                // rows past M re-read row 0 (their outputs are never stored)
                const char* base = lds + lq_a + (real ? colq : 0) * p.lrs + tt * 128 + (lane >> 4) * 16;
#pragma unroll
                for (int h = 0; h < 2; ++h) ab[sa][0][h] = *reinterpret_cast<const uint4*>(base + h * 64);
            } else {
                const char* base = lds + (real ? lq_a + colq * p.lrs + tt * 128 : lq_z) + (lane >> 4) * 16;
#pragma unroll
                for (int h = 0; h < 2; ++h) ab[sa][0][h] = *reinterpret_cast<const uint4*>(base + (real ? h * 64 : 0));
            }
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
        // the one scale per column is loaded once, before the loop; STS stages them
        if constexpr (ONE || STS) return;
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
        if constexpr (STS && decltype(prefetch)::value) {
            // the next pass's buffer (its activations are read during this one)
            stage_commit(it + 1);
            stage_issue(it + 2);
        }
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const int t = ta + it * D + s;
            uint32_t sc[CPW][NS];
            if constexpr (STS && !ONE) {
                const char* const sbase = lds + lw + 16 + (it & 1) * st_buf + st_ab + colq * 2;
                const int g0 = gfirst(ta + it * D);
#pragma unroll
                for (int c = 0; c < CPW; ++c)
#pragma unroll
                    for (int j = 0; j < NS; ++j)
                        sc[c][j] = *reinterpret_cast<const uint16_t*>(sbase + (c * NGP + graw(t, j) - g0) * 32);
            } else {
#pragma unroll
                for (int c = 0; c < CPW; ++c)
#pragma unroll
                    for (int j = 0; j < NS; ++j) sc[c][j] = sb[s][c][j];
            }
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
                if (h == 1) {
                    if constexpr (ST) load_a_st(s, it + 1, s);
                    else load_a(s % DA, t + DA);
                }
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
    uint4 xw[QW > 0 ? QW : 1];
    if constexpr (QW > 0) {
        // every wave reads the whole row (L2-resident after the first reads):
        // its absmax then needs no other wave's, so no barrier
        const auto rx = make_rsrc(p.X, static_cast<uint32_t>(p.K * 2));
#pragma unroll
        for (int i = 0; i < QW; ++i) {
            const int c = lane + 64 * i;
            xw[i] = buf_load16(rx, c < (p.K >> 3) ? static_cast<uint32_t>(c * 16) : kOOB);
        }
    } else if constexpr (QF) {
        // raw buffer loads, chunks outside the range reading zero: no
        // per-lane branches, so the waits below can count the weight loads
        // issued after these instead of draining everything
        const auto rx = make_rsrc(p.X, static_cast<uint32_t>(((p.M - 1) * p.ldx + p.K) * 2));
#pragma unroll
        for (int m = 0; m < QM; ++m)
#pragma unroll
            for (int i = 0; i < QI; ++i) {
                const int c = lane + 64 * i;
                const bool ok = m < p.M && i < p.qcpr && c < nch;
                xv[m][i] = buf_load16(rx, ok ? static_cast<uint32_t>((m * p.ldx + k0 + 8 * c) * 2) : kOOB);
            }
    }
    uint32_t ws1[CPW];   // ONE: the scale of each column block's columns of this lane
    // QF: issued by every wave (an idle wave's range is empty, so its loads
    // read zeros through empty descriptors) -- under a branch the wait for
    // the X rows below would also wait for the whole weight ring.
    if (QF || busy) {
        if constexpr (STS) stage_issue(0);
#pragma unroll
        for (int s = 0; s < D; ++s) load_slot(s, ta + s);
    }
    // QF: every load above is issued before the quant's first use of X (left
    // to itself the scheduler starts the absmax first and the ring waits for
    // the rows to arrive)
    if constexpr (QF) __builtin_amdgcn_sched_barrier(0);
    if constexpr (ONE) {
        const auto rs = make_rsrc(p.S, p.s_bytes);
#pragma unroll
        for (int c = 0; c < CPW; ++c) ws1[c] = buf_load_u16(rs, so[c]);
    }
    if constexpr (QW > 0) {
        uint32_t amax = 0u;
#pragma unroll
        for (int i = 0; i < QW; ++i) amax = max(amax, abs_bits_max8(xw[i]));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1)
            amax = max(amax, static_cast<uint32_t>(__shfl_xor(static_cast<int>(amax), off, 64)));
        amax = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(amax)));
        const uint32_t sbits = scale_from_amax(amax);
        const bool writer = cgi == 0 && rgi == 0;   // one workgroup emits a_q / a_scale
        if (wave == 0 && lane == 0) {
            reinterpret_cast<uint32_t*>(lds + lq_s)[0] = sbits;
            if (writer) p.as_out[0] = static_cast<uint16_t>(sbits);
        }
        const RowScale q = row_scale(bf16_bits_to_f32(sbits));
        // quantise this wave's own K range into its part of the LDS row
        const int c0 = k0 >> 3, c1 = k1 >> 3;
        auto emit = [&](auto fast) __attribute__((always_inline)) {
            constexpr bool F = decltype(fast)::value;
#pragma unroll
            for (int i = 0; i < QW; ++i) {
                const int c = lane + 64 * i;
                if (c >= c0 && c < c1) {
                    const uint4 v = xw[i];
                    uint2 o;
                    o.x = quant2<F>(v.x, q) | (quant2<F>(v.y, q) << 16);
                    o.y = quant2<F>(v.z, q) | (quant2<F>(v.w, q) << 16);
                    *reinterpret_cast<uint2*>(lds + lq_a + 8 * c) = o;
                    if (writer) *reinterpret_cast<uint2*>(p.aq_out + 8 * c) = o;
                }
            }
        };
        if (q.fast) emit(std::true_type{});
        else emit(std::false_type{});
    } else if constexpr (QF) {
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
        if constexpr (ST) {
            stage_commit(0);
            stage_issue(1);
#pragma unroll
            for (int s = 0; s < D; ++s) load_a_st(s, 0, s);
        } else {
            if constexpr (STS) {
                stage_commit(0);
                stage_issue(1);
            }
#pragma unroll
            for (int s = 0; s < DA; ++s) load_a(s, ta + s);
        }
        const int iters = (tb - ta + D - 1) / D;
        for (int it = 0; it + 1 < iters; ++it) pass(it, std::true_type{});
        pass(iters - 1, std::false_type{});
    }

    // Fixed-order reduction of the kw wave partials, then the epilogue.  With
    // one group the waves' int32 sums are added (exactly, so the order does
    // not matter) and folded with the column's scale once.  Wave w's rows
    // start at float w * rstride (ST: its staging area, no longer read).
    const int rstride = st_wave / 4;
    __shared__ float wsl[ONE ? C : 1];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int c = 0; c < CPW; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float* r = &red[wave * rstride + (mt * 16 + rowq + i) * C + c * 16 + colq];
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
            for (int w = 1; w < kw; ++w) isum += reinterpret_cast<const int*>(red)[w * rstride + e];
            if constexpr (DUMP) {
                const int row = e / C, col = block_of(cc / 16) * 16 + cc % 16;
                if (m0 + row < p.M && col < p.N) p.P[static_cast<int64_t>(m0 + row) * p.N + col] = isum >> 4;
            }
            return static_cast<float>(isum) * wsl[cc];
        } else {
            float sum = red[e];
            for (int w = 1; w < kw; ++w) sum += red[w * rstride + e];
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

template <int MT, int CPW, int KWMAX, int D, int GM, bool SBF16, bool DUMP, bool SWIGLU, int SA>
__global__ __launch_bounds__(64 * KWMAX) void gemm_decode_kernel(const DecodeParams p) {
    decode_body<MT, CPW, KWMAX, D, GM, SBF16, DUMP, SWIGLU, 0, SA>(p);
}


// Most waves per workgroup a variant is built for (its register budget: the
// 64-row, 4-block variant needs 256 VGPRs at 2 waves per SIMD).
constexpr int kwmax_for(int mt, int cpw, int d) {
    // one 16-row tile of one column block with a 4-deep ring fits 16 waves (128 VGPRs)
    return mt == 1 ? (cpw >= 4 ? 8 : (cpw == 1 && d <= 4 ? 16 : 12)) : (mt == 2 || cpw <= 2 ? 8 : 4);
}

// MODE: 0 = plain, 1 = plain with partial dump, 2 = SwiGLU epilogue.
// Largest LDS a decode workgroup is launched with.
constexpr size_t kDecodeLdsMax = 64 * 1024;

// SA > 0: the staged variant (its launcher refuses an area past kDecodeLdsMax).
template <int MT, int CPW, int D, int GM, int MODE, int SA = 0>
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
        const size_t lds = SA > 0 ? static_cast<size_t>(w) * st_wave_bytes(p.M, CPW, GM, D)
                                  : static_cast<size_t>(w) * 16 * MT * 16 * CPW * sizeof(float);
        if (SA > 0 && (p.M > 2 * SA || lds > kDecodeLdsMax)) return hipErrorInvalidValue;
        if (sbf16) gemm_decode_kernel<MT, CPW, KWM, D, GM, true, DUMP, SWIGLU, SA><<<grid, block, lds, stream>>>(q);
        else gemm_decode_kernel<MT, CPW, KWM, D, GM, false, DUMP, SWIGLU, SA><<<grid, block, lds, stream>>>(q);
        return hipGetLastError();
    }
}

// Group mode: one group over all of K -> 4; otherwise by group stride: 64 ->
// 0; 128 -> 3; 128 * 2^s, s >= 1 -> 1; anything else -> 2.
inline int group_mode(int spg, int ng) {
    if (ng == 1) return 4;
    if (spg == 1) return 0;
    if (spg == 2) return 3;
    if (spg % 2 == 0 && ((spg / 2) & (spg / 2 - 1)) == 0) return 1;
    return 2;
}

template <int MT, int CPW, int D, int MODE, int SA = 0>
hipError_t launch_v(const DecodeParams& p, int kw, bool sbf16, hipStream_t stream) {
    switch (group_mode(p.spg, p.NG)) {
        case 0: return launch_g<MT, CPW, D, 0, MODE, SA>(p, kw, sbf16, stream);
        case 1: return launch_g<MT, CPW, D, 1, MODE, SA>(p, kw, sbf16, stream);
        case 3: return launch_g<MT, CPW, D, 3, MODE, SA>(p, kw, sbf16, stream);
        case 4: return launch_g<MT, CPW, D, 4, MODE, SA>(p, kw, sbf16, stream);
        default: return launch_g<MT, CPW, D, 2, MODE, SA>(p, kw, sbf16, stream);
    }
}

// The staged variants (gemm_decode_staged.hip): one 16-row tile of M <= 8
// rows, D = 4, CPW 1 or 2 (2 for the SwiGLU epilogue).
template <int MODE>
hipError_t dispatch_staged(const DecodeParams& p, const DecodeConfig& c, bool sbf16, hipStream_t s);

// Whether the staged variant serves M rows with kw waves of cpw column blocks.
inline bool staged_fits(int64_t M, int cpw, int gm, int kw) {
    return M >= 1 && M <= 8 && (cpw == 1 || cpw == 2) &&
           static_cast<size_t>(kw) * st_wave_bytes(static_cast<int>(M), cpw, gm, 4) <= kDecodeLdsMax;
}

}  // namespace dec
}  // namespace w4a8
