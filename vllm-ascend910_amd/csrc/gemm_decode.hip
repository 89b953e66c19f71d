// Decode-shaped W4A8 GEMM (M <= 64): the launch plans, the per-tile variants
// and the fused quant + GEMM of one row.  The kernel body and its design are
// in decode_kernel.h; the staged-activation variants are built in
// gemm_decode_staged.hip.
#include <algorithm>
#include <type_traits>

#include "decode_kernel.h"

namespace w4a8 {
namespace {

using namespace dec;

template <int KWMAX, int GM, bool SBF16, int QW>
__global__ __launch_bounds__(64 * KWMAX) void linear_decode_kernel(const DecodeParams p) {
    decode_body<1, 2, KWMAX, 4, GM, SBF16, false, false, 1, 0, QW>(p);
}

int gcd_i(int a, int b) {
    while (b) {
        const int t = a % b;
        a = b;
        b = t;
    }
    return a;
}

// The variants that are built: (MT, D, CPW); the SwiGLU epilogue needs an
// even CPW.
template <int MODE>
hipError_t dispatch(const DecodeParams& p, const DecodeConfig& c, bool sbf16, hipStream_t s) {
    // c.MT > 0: workgroups of 16 * c.MT rows, gridDim.y of them
    const int mt = c.MT > 0 ? std::min(c.MT, (p.M + 15) / 16) : (p.M + 15) / 16;
    if (c.STAGE) return dispatch_staged<MODE>(p, c, sbf16, s);
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
    // rows of up to 8192 elements: every wave reads the whole row (16 chunks per lane at most)
    if (p.K <= 64 * 8 * 10)
        linear_decode_kernel<KWM, GM, SBF16, 10><<<dim3(static_cast<unsigned>(p.cgroups)), dim3(64 * kw), lds, stream>>>(p);
    else if (p.K <= 64 * 8 * 16)
        linear_decode_kernel<KWM, GM, SBF16, 16><<<dim3(static_cast<unsigned>(p.cgroups)), dim3(64 * kw), lds, stream>>>(p);
    else
        linear_decode_kernel<KWM, GM, SBF16, 0><<<dim3(static_cast<unsigned>(p.cgroups)), dim3(64 * kw), lds, stream>>>(p);
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
    // One row only: every workgroup quantises the row again (each wave its
    // own K range; up to 8192 elements each wave reads the whole row for the
    // absmax, longer rows meet in LDS), so the quant work is repeated per
    // column group.  Measured on MI355X against the quant kernel + GEMM pair
    // (graph replays, cold weights): qkv 7.6 against 8.6 us, o 7.1 against
    // 8.1, gate_up 25.9 against 28.0, down_proj (long K, eight waves of 27
    // tiles) 19.3 against 19.5 -- and one launch fewer where the linear runs
    // inside a captured graph.  What remains over the GEMM alone (qkv 5.7 us)
    // is the round trip of the cold bf16 row, which the pair pays in its quant
    // kernel.  The four-row variant of the LDS-exchange prologue lost 2 us on
    // qkv and o at M=4.
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
    // reduction rows, quantised rows, zero block, absmax, scale bits, then per
    // wave the staged group scales (a dump slot and two pass buffers)
    const int gm = group_mode(f.p.spg, f.p.NG);
    const int sts = gm == 4 ? 0 : 16 + 2 * 2 * st_pass_groups(gm, 4) * 32;
    f.lds = static_cast<size_t>(f.kw) * 16 * 32 * 4 + static_cast<size_t>(f.qm) * f.p.lrs + 64 + f.kw * 16 + 16 +
            static_cast<size_t>(f.kw) * sts;
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
        // -- two up to 4 rows (staged: gate_up M=4 24.5 against 24.7 us; a
        // single row's fused-quant plan, the same split, needs a wave's K
        // range to fit its prologue's registers).
        if (mt == 1) c.KW = M <= 4 ? 2 : 1;
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
    // Up to 8 rows in one tile: staged activations and scales wherever the
    // waves' LDS areas fit (measured on MI355X, cold, G=128, M=1/4/8:
    // down_proj 19.7/17.0/18.8 -> 14.8/15.8/17.3 us, o_proj 6.0/5.8 ->
    // 5.1/5.4 us, qkv_proj 6.3/6.4 -> 5.8/5.9 us, gate_up 26.2/25.0/26.0 ->
    // 24.5/24.5/25.7 us; qkv and o at 8 rows keep ten per-tile waves, which
    // the 64 KB area cap would cut to six).
    if (c.MT == 0 && mt == 1 && c.D == 4) {
        const int gm = group_mode(static_cast<int>(geom::group_stride(group) / 64),
                                  static_cast<int>(geom::num_groups(K, group)));
        c.STAGE = staged_fits(M, c.CPW, gm, c.KW) ? 1 : 0;
    }
    return c;
}

// The plans without the split prefill tiles.
DecodeConfig base_config(int64_t M, int64_t N, int64_t K, int64_t group) {
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

}  // namespace

DecodeConfig decode_config(int64_t M, int64_t N, int64_t K, int64_t group) {
    DecodeConfig c = base_config(M, N, K, group);
    const int64_t KT = geom::k_tiles(K, group);
    // Narrow N with long K past 32 rows at group stride 128: one 64-row tile
    // of the prefill kernel's 128 x 32 wave tiles, K split so that the
    // workgroups cover about 15/16 of the CUs once (down_proj on MI355X: six
    // splits of 36 steps, 240 workgroups).  Cold, us, against the wide layout
    // split six ways: M=48 27.5 -> 24.0, M=64 28.8 -> 25.3; at 24 and 32 rows
    // it loses (23.7 -> 25.9, 24.3 -> 26.1), as it does on qkv/o at 24-64 rows
    // (short K: 12.6 -> 14.8 on qkv M=64 at its best split).
    if (c.WIDE && c.SPLITS > 1 && M > 32 && geom::group_stride(group) == 128) {
        const int64_t tn = geom::ceil_div(N, int64_t{128});
        const int64_t target = device_cu_count() * 15 / 16;
        const int64_t s = std::min<int64_t>({(target + tn / 2) / tn, KT / 8, int64_t{16}});
        if (s > 1) c.PSPLIT = static_cast<int>(s);
    }
    return c;
}

int64_t decode_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group) {
    const DecodeConfig c = decode_config(M, N, K, group);
    const int64_t fb = c.WIDE && c.SPLITS > 1 ? wide_workspace_bytes(M, N, K, group, c.SPLITS) : 0;
    return c.PSPLIT ? std::max(fb, prefill_split_workspace_bytes(M, N, K, group, c.PSPLIT)) : fb;
}

hipError_t launch_gemm_decode_cfg(const GemmArgs& a, const DecodeConfig& cfg, hipStream_t stream) {
    // the split prefill tiles have no SwiGLU pairs and no partial dump: those
    // calls take the fallback plan held in the other fields
    if (cfg.PSPLIT && !a.swiglu && !a.partials) return launch_gemm_prefill_split(a, cfg.PSPLIT, stream);
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
