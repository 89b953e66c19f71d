// Decode-shaped W4A8 GEMM for up to 64 rows with the activations shared
// through LDS (the decode heuristic sends it 9-64 rows on wide N, and on
// narrow N with long K).
//
// Same arithmetic as gemm_decode.hip (exact int32 per group on
// v_mfma_i32_16x16x64_i8, fp32 fold with the group scale, token scale at the
// end).  The decode kernel gives every wave all rows and its own K range, so
// every workgroup streams the whole activation block from L2 for its few
// column blocks: at 64 rows on gate_up that is twice the weight bytes.  Here a
// workgroup of kWN column waves covers kWN * kCPW column blocks; its waves
// share each activation tile (16 * kMT rows x 128 K), staged once into LDS
// (double-buffered, one barrier per tile) and read from there as MFMA
// operands.  The staging loads run kRA tiles ahead in registers and the
// weights stream straight to registers in a kD-deep ring.
//
// A workgroup walks one K range of a group-aligned split (blockIdx.y).  With
// one split it writes bf16 directly and the accumulation order per output is
// the decode kernel's with one K wave.  With several splits each workgroup
// writes its fp32 sums (before the token scale) to the workspace and
// wide_reduce_kernel adds the splits in index order, applies the token scale
// and rounds to bf16 -- the order the decode kernel's in-workgroup K split
// reduces its waves in.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "kgeom.h"
#include "launch.h"

namespace w4a8 {
namespace {

constexpr int kALS = 128 + 16;         // LDS row stride of a staged activation tile (bytes)
constexpr uint32_t kOOBW = 0x80000000u;
constexpr int kWaves = 4;              // column waves per workgroup
constexpr int kMaxSplits = 16;         // K splits over workgroups, at most

struct WideParams {
    const int8_t* A;
    int64_t lda;
    const uint16_t* a_scale;
    const uint4* W;
    const uint16_t* S;
    uint16_t* Y;
    int64_t ldy;
    int32_t* P;        // optional partial dump [NG, M, N]
    float* R;          // splits > 1: fp32 sums [splits, M, ldr]
    int64_t ldr;       // NB * 16
    int M, N, KT, NG, NB;
    int up_nb;         // SWIGLU: column blocks per half
    int nslab, spg, gshift;
    int unit, units, splits;   // K split: tiles per group-aligned unit, units, workgroups along K
    uint32_t a_bytes, w_bytes, s_bytes;
};

// f(integral_constant<int, J>) for J = B .. E-1, in order.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// GM: the group modes of gemm_decode.hip (0: stride 64, 3: stride 128,
// 1: stride 128 * 2^gshift, 2: any other stride, 4: one group over all of K).
// Mode 4 folds once after the K loop; with K split over workgroups it writes
// the int32 sums instead, which wide_reduce_kernel adds exactly and folds.
// kMT 16-row tiles, kWN column waves, kCPW 16-column blocks per wave, kD
// weight ring depth, kRA activation tiles in flight.
template <int kMT, int kWN, int kCPW, int kD, int kRA, int GM, bool SBF16, bool DUMP, bool SWIGLU>
__global__ __launch_bounds__(64 * kWN) void gemm_wide_kernel(const WideParams p) {
    static_assert(!(SWIGLU && DUMP), "the SwiGLU variant dumps nothing");
    constexpr int CG = SWIGLU ? kCPW / 2 : kCPW;   // output column blocks per wave
    constexpr int NS = (GM == 1 || GM == 3 || GM == 4) ? 1 : 2;
    constexpr bool ONE = GM == 4;
    // kDW: group scales loaded as the aligned dword that holds the lane's
    // 16-bit scale (32 and 64 rows: gate_up M=32 33.6 -> 32.0 us, M=64
    // 40.3 -> 39.5, down M=64 31.9 -> 30.6; 16 rows lose ~0.4 us with it).
    // A ring of 16-bit loads makes the compiler zero-extend each loaded
    // value on the loop latch, a copy that waits for the loads just issued.
    constexpr bool kDW = kMT >= 2 && !ONE;
    // Unroll: every ring slot index is static; with kDW a slot's scale lives
    // in two registers in turn (the next load is issued before the last one
    // is used), so a multiple of 2 kD steps needs no copy on the loop latch.
    constexpr int kDU = kDW ? 2 * kD : kD;
    constexpr int U = kDU > kRA ? kDU : kRA;
    static_assert(U % kD == 0 && U % kRA == 0 && U % 2 == 0, "ring depths must divide the unroll");
    constexpr int kATile = 16 * kMT * kALS;
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

    // Token scales of the rows: requested here, parked in LDS after the K
    // loop (loads issued in the epilogue would add a memory round trip to
    // the tail of every call).
    __shared__ uint32_t tsc[16 * kMT];
    uint32_t ts_bits = 0;
    if (tid < 16 * kMT && tid < p.M) ts_bits = p.a_scale[tid];

    // This workgroup's K range [ta, tb): group-aligned units split evenly
    // (the host keeps splits <= units, so every range is non-empty).
    const int ks = static_cast<int>(blockIdx.y);
    const int ua = (ks * p.units) / p.splits;
    const int ub = ((ks + 1) * p.units) / p.splits;
    const int ta = ua * p.unit;
    const int tb = min(p.KT, ub * p.unit);
    const int nit = tb - ta;

    uint32_t wo[kCPW], so[kCPW];
    const uint32_t ssh = kDW ? (colq & 1) * 16u : 0u;   // column colq's half of a scale dword
#pragma unroll
    for (int c = 0; c < kCPW; ++c) {
        const uint32_t nb = static_cast<uint32_t>(min(block_of(c), p.NB - 1));
        wo[c] = nb * static_cast<uint32_t>(p.KT) * 1024u + lane * 16u;
        so[c] = (nb * static_cast<uint32_t>(p.NG) * 16u + (kDW ? (colq & ~1) : colq)) * 2u;
    }
    // Staging: 16 * kMT rows x 128 K = 128 * kMT units of 16 bytes, NU per
    // lane; rows past M read zero.  With fewer units than lanes (one row
    // tile) the waves past the units stage nothing (a wave-uniform test).
    constexpr int kUnits = 128 * kMT;
    constexpr int NU = (kUnits + 64 * kWN - 1) / (64 * kWN);
    static_assert(NU * 64 * kWN == kUnits || (NU == 1 && kUnits % 64 == 0), "staging units per wave");
    constexpr bool kAllStage = kUnits >= 64 * kWN;
    const bool stager = kAllStage || wn * 64 < kUnits;
    uint32_t sg[NU];
    int sl[NU];
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        const int u = kAllStage ? lane + 64 * (wn + kWN * j) : min(lane + 64 * wn, kUnits - 1);
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

    uint4 ra[kRA][NU];
    auto stage_load = [&](int t, uint4 (&r)[NU]) {
        if (!kAllStage && !stager) return;
        // tiles past the end stage the last tile again (nothing reads them)
        const auto rs = make_rsrc_at(p.A, static_cast<uint32_t>(min(t, p.KT - 1)) * 128u, p.a_bytes);
#pragma unroll
        for (int j = 0; j < NU; ++j) r[j] = buf_load16(rs, sg[j]);
    };
    auto stage_store = [&](int buf, const uint4 (&r)[NU]) {
        if (!kAllStage && !stager) return;
#pragma unroll
        for (int j = 0; j < NU; ++j) *reinterpret_cast<uint4*>(&la[buf][sl[j]]) = r[j];
    };

    uint4 wb[kD][kCPW];
    uint32_t sb[kD][kCPW][NS];
    auto load_slot = [&](int s, int t) {
        const auto rw = make_rsrc_at(p.W, static_cast<uint32_t>(min(t, p.KT - 1)) * 1024u, t < tb ? p.w_bytes : 0u);
#pragma unroll
        for (int c = 0; c < kCPW; ++c) wb[s][c] = buf_load16_nt(rw, wo[c]);
        if constexpr (ONE) return;   // the one scale per column is loaded once
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            const auto rs = make_rsrc_at(p.S, static_cast<uint32_t>(gend(min(t, p.KT - 1), j)) * 32u, p.s_bytes);
#pragma unroll
            for (int c = 0; c < kCPW; ++c) sb[s][c][j] = kDW ? buf_load_u32(rs, so[c]) : buf_load_u16(rs, so[c]);
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

    auto fold = [&](int g, const float (&sc)[kCPW][NS], int j) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < kCPW; ++c) {
            const float ws = sc[c][j];
#pragma unroll
            for (int mt = 0; mt < kMT; ++mt) {
                if constexpr (DUMP) {
                    const int col = block_of(c) * 16 + colq;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int row = mt * 16 + rowq + i;
                        if (row < p.M && col < p.N && g < p.NG)
                            p.P[(static_cast<int64_t>(g) * p.M + row) * p.N + col] = P[mt][c][i] >> 4;
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mt][c][i] += static_cast<float>(P[mt][c][i]) * ws;
                if constexpr (GM == 1 || GM == 2) P[mt][c] = v4i{0, 0, 0, 0};
            }
        }
    };

    // ---- prologue: tiles ta .. ta+kRA-1 in flight to the staging registers,
    // the weight ring filled, tile ta staged in buffer 0
    stage_load(ta, ra[0]);
#pragma unroll
    for (int s = 0; s < kD; ++s) load_slot(s, ta + s);
    uint32_t ws1[kCPW];   // ONE: this lane's column scale per column block
    if constexpr (ONE) {
        const auto rs = make_rsrc(p.S, p.s_bytes);
#pragma unroll
        for (int c = 0; c < kCPW; ++c) ws1[c] = buf_load_u16(rs, so[c]);
    }
#pragma unroll
    for (int r = 1; r < kRA; ++r) stage_load(ta + r, ra[r]);
    stage_store(0, ra[0]);
    __syncthreads();

    // One tile t = ta + i; J = i mod U names the ring slots and the LDS buffer.
    auto step = [&](int i, auto jc) __attribute__((always_inline)) {
        constexpr int J = decltype(jc)::value;
        constexpr int WS = J % kD;
        const int t = ta + i;
        // the staging slot of tile t is free again (tile t is in LDS)
        stage_load(t + kRA, ra[J % kRA]);
        uint32_t raw[kCPW][NS];
#pragma unroll
        for (int c = 0; c < kCPW; ++c)
#pragma unroll
            for (int q = 0; q < NS; ++q) raw[c][q] = sb[WS][c][q];
        v4i b[kCPW][2];
#pragma unroll
        for (int c = 0; c < kCPW; ++c) unpack_tile_lane(wb[WS][c], b[c][0], b[c][1]);
        load_slot(WS, t + kD);
        // With kDW the slot's scales are converted here, once the slot's
        // next loads are issued.  The empty asm statements pin the
        // conversion: left to itself the compiler sinks it to the fold, which
        // it gathers on the loop latch, and the raw value is then copied
        // there, a copy that waits for every load in flight (the same drain
        // as hoisting it to the top of the loop, which waits for the newest
        // loads).
        float sc[kCPW][NS];
#pragma unroll
        for (int c = 0; c < kCPW; ++c)
#pragma unroll
            for (int q = 0; q < NS; ++q) {
                if constexpr (ONE) continue;
                if constexpr (kDW) asm volatile("" : "+v"(raw[c][q]));
                sc[c][q] = scale_to_f32<SBF16>(raw[c][q] >> ssh);
                if constexpr (kDW) asm volatile("" : "+v"(sc[c][q]));
            }
        // Every A operand of the tile read from LDS before the first MFMA
        // (left to itself the compiler reads the second half one operand at
        // a time, each read waited for before its MFMAs).
        const int8_t* ab = &la[J & 1][0] + colq * kALS + (lane >> 4) * 16;
        v4i av[2][kMT];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int mt = 0; mt < kMT; ++mt) av[h][mt] = *reinterpret_cast<const v4i*>(ab + mt * 16 * kALS + h * 64);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const bool fresh = GM == 0 || (GM == 3 && h == 0);
#pragma unroll
            for (int mt = 0; mt < kMT; ++mt) {
#pragma unroll
                for (int c = 0; c < kCPW; ++c)
                    P[mt][c] = mfma16(av[h][mt], b[c][h], fresh ? v4i{0, 0, 0, 0} : P[mt][c]);
            }
            if constexpr (ONE) {
                // folded once, after the K loop
            } else if constexpr (GM == 0) {
                fold(2 * t + h, sc, h);
            } else if constexpr (GM == 3) {
                if (h == 1) fold(t, sc, 0);
            } else if constexpr (GM == 1) {
                if (h == 1 && (((t + 1) & ((1 << p.gshift) - 1)) == 0 || t == p.KT - 1)) fold(t >> p.gshift, sc, 0);
            } else {
                const int sgi = 2 * t + h;
                if (sgi < p.nslab && (((sgi + 1) % p.spg) == 0 || sgi == p.nslab - 1)) fold(sgi / p.spg, sc, h);
            }
        }
        // tile t+1 into the other buffer (free: every wave finished tile t-1)
        stage_store((J + 1) & 1, ra[(J + 1) % kRA]);
        __syncthreads();
    };
    int i = 0;
    for (; i + U <= nit; i += U) static_for<0, U>([&](auto jc) { step(i + decltype(jc)::value, jc); });
    static_for<0, U - 1>([&](auto jc) {
        if (i + decltype(jc)::value < nit) step(i + decltype(jc)::value, jc);
    });

    // ---- epilogue: token scale, bf16 (or the SwiGLU pair); fp32 sums to
    // the workspace when K is split (int32 sums for one group)
    if constexpr (ONE) {
        if (p.splits == 1) {
            float sc1[kCPW][NS];
#pragma unroll
            for (int c = 0; c < kCPW; ++c) sc1[c][0] = scale_to_f32<SBF16>(ws1[c] >> ssh);
            fold(0, sc1, 0);
        }
    }
    if (tid < 16 * kMT) tsc[tid] = ts_bits;
    __syncthreads();
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int row = mt * 16 + rowq + q;
            if (row >= p.M) continue;
            if constexpr (SWIGLU) {
                const float ts = bf16_bits_to_f32(tsc[row]) * 0.0625f;
#pragma unroll
                for (int c = 0; c < CG; ++c) {
                    const int col = block_of(c) * 16 + colq;
                    if (col < p.up_nb * 16)
                        p.Y[static_cast<int64_t>(row) * p.ldy + col] =
                            static_cast<uint16_t>(swiglu_bf16_bits(acc[mt][c][q] * ts, acc[mt][c + CG][q] * ts));
                }
            } else if (p.splits > 1) {
                float* r = p.R + (static_cast<int64_t>(ks) * p.M + row) * p.ldr;
#pragma unroll
                for (int c = 0; c < kCPW; ++c) {
                    const int col = block_of(c) * 16 + colq;
                    if (col < p.N) {
                        if constexpr (ONE) reinterpret_cast<int*>(r)[col] = P[mt][c][q];
                        else r[col] = acc[mt][c][q];
                    }
                }
            } else {
                const float ts = bf16_bits_to_f32(tsc[row]) * 0.0625f;
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

// y[m, n] = bf16((R[0, m, n] + R[1, m, n] + ...) * token scale), four
// columns per thread; R rows are ldr (a multiple of 16) floats apart and
// columns from N to ldr are never written.  ONE (a single group over K): R
// holds int32 sums, added exactly and then folded with the column scale
// (s_tiles of one group are indexed by column), and the dump P, if given,
// receives the group's partial.
template <bool ONE, bool SBF16>
__global__ __launch_bounds__(256) void wide_reduce_kernel(const float* __restrict__ R, int64_t ldr,
                                                          const uint16_t* a_scale, uint16_t* Y, int64_t ldy, int M,
                                                          int N, int splits, const uint16_t* S, int32_t* P) {
    const int n4 = static_cast<int>(ldr >> 2);
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= static_cast<int64_t>(M) * n4) return;
    const int row = static_cast<int>(idx / n4);
    const int col = static_cast<int>(idx - static_cast<int64_t>(row) * n4) * 4;
    if (col >= N) return;
    const uint32_t tsb = a_scale[row];   // requested with the sums, not after them
    const int64_t plane = static_cast<int64_t>(M) * ldr;
    const float* r = R + static_cast<int64_t>(row) * ldr + col;
    // all loads first (one memory latency, not one per split), then the sum
    // in split order
    float4 v[kMaxSplits];
#pragma unroll
    for (int k = 0; k < kMaxSplits; ++k)
        v[k] = k < splits ? *reinterpret_cast<const float4*>(r + k * plane) : make_float4(0.f, 0.f, 0.f, 0.f);
    float4 s = v[0];
    if constexpr (ONE) {
        int4 is = *reinterpret_cast<const int4*>(&v[0]);
#pragma unroll
        for (int k = 1; k < kMaxSplits; ++k) {
            if (k < splits) {
                const int4 t = *reinterpret_cast<const int4*>(&v[k]);
                is.x += t.x;
                is.y += t.y;
                is.z += t.z;
                is.w += t.w;
            }
        }
        const int iv[4] = {is.x, is.y, is.z, is.w};
        float sv[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int cc = min(col + c, N - 1);
            sv[c] = static_cast<float>(iv[c]) * scale_to_f32<SBF16>(S[cc]);
            if (P != nullptr && col + c < N) P[static_cast<int64_t>(row) * N + col + c] = iv[c] >> 4;
        }
        s = make_float4(sv[0], sv[1], sv[2], sv[3]);
    } else {
#pragma unroll
        for (int k = 1; k < kMaxSplits; ++k) {
            if (k < splits) {
                s.x += v[k].x;
                s.y += v[k].y;
                s.z += v[k].z;
                s.w += v[k].w;
            }
        }
    }
    const float ts = bf16_bits_to_f32(tsb) * 0.0625f;
    const uint32_t lo = f32_to_bf16_bits(s.x * ts) | (f32_to_bf16_bits(s.y * ts) << 16);
    const uint32_t hi = f32_to_bf16_bits(s.z * ts) | (f32_to_bf16_bits(s.w * ts) << 16);
    uint16_t* y = Y + static_cast<int64_t>(row) * ldy + col;
    if (col + 4 <= N && (reinterpret_cast<uintptr_t>(y) & 7u) == 0) {
        *reinterpret_cast<uint2*>(y) = make_uint2(lo, hi);
    } else {
        const uint16_t v[4] = {static_cast<uint16_t>(lo), static_cast<uint16_t>(lo >> 16), static_cast<uint16_t>(hi),
                               static_cast<uint16_t>(hi >> 16)};
        for (int c = 0; c < 4 && col + c < N; ++c) y[c] = v[c];
    }
}

int group_mode_of(int spg, int ng) {
    if (ng == 1) return 4;
    if (spg == 1) return 0;
    if (spg == 2) return 3;
    if (spg % 2 == 0 && ((spg / 2) & (spg / 2 - 1)) == 0) return 1;
    return 2;
}

int gcd_w(int a, int b) {
    while (b) {
        const int t = a % b;
        a = b;
        b = t;
    }
    return a;
}

template <int kMT, int kCPW, int kD, int kRA, int GM, bool DUMP, bool SWIGLU>
hipError_t launch_g(const WideParams& p, int cgroups, bool sbf16, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(cgroups), static_cast<unsigned>(p.splits)), block(64 * kWaves);
    if (sbf16) gemm_wide_kernel<kMT, kWaves, kCPW, kD, kRA, GM, true, DUMP, SWIGLU><<<grid, block, 0, s>>>(p);
    else gemm_wide_kernel<kMT, kWaves, kCPW, kD, kRA, GM, false, DUMP, SWIGLU><<<grid, block, 0, s>>>(p);
    return hipGetLastError();
}

template <int kMT, int kCPW, int kD, int kRA, bool DUMP, bool SWIGLU>
hipError_t launch_gm(const WideParams& p, int cgroups, bool sbf16, hipStream_t s) {
    switch (group_mode_of(p.spg, p.NG)) {
        case 4: return launch_g<kMT, kCPW, kD, kRA, 4, DUMP, SWIGLU>(p, cgroups, sbf16, s);
        case 0: return launch_g<kMT, kCPW, kD, kRA, 0, DUMP, SWIGLU>(p, cgroups, sbf16, s);
        case 1: return launch_g<kMT, kCPW, kD, kRA, 1, DUMP, SWIGLU>(p, cgroups, sbf16, s);
        case 3: return launch_g<kMT, kCPW, kD, kRA, 3, DUMP, SWIGLU>(p, cgroups, sbf16, s);
        default: return launch_g<kMT, kCPW, kD, kRA, 2, DUMP, SWIGLU>(p, cgroups, sbf16, s);
    }
}

// Parameters of one call; splits is clamped to the group-aligned units (and
// to 1 for the SwiGLU epilogue, which needs the whole sum).
WideParams make_wide_params(const GemmArgs& a, int splits) {
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
    // lcm(2, spg) slabs in tiles; any tile for a single group (int32 sums)
    p.unit = p.NG == 1 ? 1 : (2 * p.spg / gcd_w(2, p.spg)) / 2;
    p.units = (p.KT + p.unit - 1) / p.unit;
    p.splits = a.swiglu ? 1 : std::max(1, std::min({splits, p.units, kMaxSplits}));
    p.ldr = static_cast<int64_t>(p.NB) * 16;
    p.a_bytes = static_cast<uint32_t>((a.M - 1) * a.lda + geom::kpad(a.K, a.group));
    p.w_bytes = static_cast<uint32_t>(p.NB * static_cast<int64_t>(p.KT) * geom::kTileBytes);
    p.s_bytes = static_cast<uint32_t>(p.NB * static_cast<int64_t>(p.NG) * 16 * 2);
    return p;
}

int64_t split_bytes(const WideParams& p) {
    return p.splits > 1 ? static_cast<int64_t>(p.splits) * p.M * p.ldr * 4 : 0;
}

// One call with an explicit layout: kMT row tiles, kCPW column blocks per
// wave, ring depths kD / kRA, p.splits workgroups along K.
template <int kMT, int kCPW, int kD, int kRA>
hipError_t launch_wide_v(const GemmArgs& a, WideParams p, hipStream_t stream) {
    if (a.M <= 0 || a.M > 16 * kMT) return hipErrorInvalidValue;
    if (a.swiglu && kCPW % 2 != 0) return hipErrorInvalidValue;
    const int64_t need = split_bytes(p);
    if (need > 0) {
        if (a.workspace == nullptr || a.workspace_bytes < need) return hipErrorInvalidValue;
        p.R = static_cast<float*>(a.workspace);
    }
    const int per_wg = kWaves * kCPW;
    const int64_t cg = a.swiglu ? geom::ceil_div(p.up_nb, per_wg / 2) : geom::ceil_div(p.NB, per_wg);
    const int c = static_cast<int>(cg);
    hipError_t e;
    if (a.swiglu) {
        if constexpr (kCPW % 2 == 0) e = launch_gm<kMT, kCPW, kD, kRA, false, true>(p, c, a.scale_bf16, stream);
        else return hipErrorInvalidValue;
    } else if (a.partials) e = launch_gm<kMT, kCPW, kD, kRA, true, false>(p, c, a.scale_bf16, stream);
    else e = launch_gm<kMT, kCPW, kD, kRA, false, false>(p, c, a.scale_bf16, stream);
    if (e != hipSuccess || p.splits == 1) return e;
    return launch_split_reduce(p.R, p.ldr, p.a_scale, p.Y, p.ldy, p.M, p.N, p.splits, p.NG == 1, a.scale_bf16, p.S,
                               p.P, stream);
}

}  // namespace

hipError_t launch_split_reduce(const float* R, int64_t ldr, const uint16_t* a_scale, uint16_t* Y, int64_t ldy, int M,
                               int N, int splits, bool one, bool sbf16, const uint16_t* S, int32_t* P,
                               hipStream_t stream) {
    const int64_t n = static_cast<int64_t>(M) * (ldr / 4);
    const dim3 rg(static_cast<unsigned>((n + 255) / 256));
    if (one) {
        if (sbf16) wide_reduce_kernel<true, true><<<rg, 256, 0, stream>>>(R, ldr, a_scale, Y, ldy, M, N, splits, S, P);
        else wide_reduce_kernel<true, false><<<rg, 256, 0, stream>>>(R, ldr, a_scale, Y, ldy, M, N, splits, S, P);
    } else {
        wide_reduce_kernel<false, false><<<rg, 256, 0, stream>>>(R, ldr, a_scale, Y, ldy, M, N, splits, nullptr,
                                                                  nullptr);
    }
    return hipGetLastError();
}

// The layouts launch_gemm_wide builds: (row tiles, column blocks per wave,
// weight ring, activation ring), measured best for their row counts on
// MI355X at the QwQ-32B shapes.
hipError_t launch_gemm_wide(const GemmArgs& a, int layout, int splits, hipStream_t stream) {
    const WideParams p = make_wide_params(a, splits);
    switch (layout) {
        case kWide1x2: return launch_wide_v<1, 2, 2, 4>(a, p, stream);
        case kWide2x2: return launch_wide_v<2, 2, 2, 2>(a, p, stream);
        case kWide4x2: return launch_wide_v<4, 2, 2, 4>(a, p, stream);
        case kWide1x1: return launch_wide_v<1, 1, 4, 4>(a, p, stream);
        case kWide2x1: return launch_wide_v<2, 1, 4, 4>(a, p, stream);
        case kWide4x1: return launch_wide_v<4, 1, 2, 2>(a, p, stream);
        default: return hipErrorInvalidValue;
    }
}

bool wide_layout_pairs(int layout) { return layout == kWide1x2 || layout == kWide2x2 || layout == kWide4x2; }

int64_t wide_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group, int splits) {
    GemmArgs a{};
    a.M = M;
    a.N = N;
    a.K = K;
    a.group = group;
    a.lda = geom::kpad(K, group);
    return split_bytes(make_wide_params(a, splits));
}

}  // namespace w4a8
