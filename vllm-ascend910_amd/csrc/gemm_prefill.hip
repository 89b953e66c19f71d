// Prefill-shaped W4A8 GEMM (M > 64): int8 MFMA bound.
//
// Same arithmetic as the decode path (gemm_decode.hip): exact int32 per group,
// fp32 fold with the group scale, token scale at the end.
//
// Tiling.  A 256-thread workgroup (4 waves, one per SIMD; two workgroups
// share a CU, so every SIMD runs two independent waves) computes a
// BM x BN = 128 x 128 output tile; wave (wm, wn) owns rows wm*64..+64 and
// columns wn*64..+64 as 2 x 2 blocks of v_mfma_i32_32x32x32_i8.  The K loop
// walks 128-K steps (one repacked weight tile row):
//   * activations: each step's A[128 rows][128 K] int8 goes from memory
//     straight into one of four LDS buffers (16-byte buffer loads to LDS,
//     three steps ahead, no registers on the way), in a swizzled layout
//     that keeps the MFMA operand reads free of bank conflicts; one barrier per
//     step, after a wait that leaves the two newest steps' loads in flight;
//   * weights: every wave loads its own 64 columns straight from the repacked
//     tiles into registers, DW steps ahead.  For a 32x32x32 B operand lane
//     (column c, half hh) and slab s the natural K order k = 32s + 16hh + [0,16)
//     is held by repacked lane (c%16) + 16*(2*(s%2) + hh), bytes 8*(s/2)..+8,
//     so each lane needs exactly two 16-byte chunks per step and unpacks them
//     with two AND/shift operations per 8 codes -- no shuffles.
// All global reads are raw buffer loads (SGPR descriptor + 32-bit offset):
// rows past M and column blocks past N read as zero, and per-lane addresses
// cost one VGPR.  The per-group fold (acc += float(16*P) * w_scale, a convert
// and an FMA per output element and group: 8 VALU instructions per MFMA at
// group 128, 3 more unpack the weights) takes more VALU cycles (4 per wave64
// instruction) than the MFMAs take matrix-core cycles (32 each), so this
// kernel is bound by VALU issue and MFMA/VALU overlap rather than by the
// matrix cores.  At group 128 each row block's fold is interleaved with the
// other row block's MFMAs (one MFMA, eight fold instructions), so one wave
// keeps both pipes busy.
#include <algorithm>

#include "common.h"
#include "kgeom.h"
#include "launch.h"

namespace w4a8 {
namespace {

// Tile BM x kBN: BM = 128 (2 x 2 waves of 64 x 64, two workgroups per CU) or
// BM = 64 (1 x 2 waves, four workgroups per CU: twice as many tiles, for
// prefills whose 128-row tiles would load the CUs unevenly; prefill_tile_rows).
constexpr int kWN = 2;                     // waves across the tile's columns
constexpr int kBN = 64 * kWN;
constexpr int kNA = 4;                     // 16-byte A chunks per lane per step (BM * 8 / threads)
constexpr int kNB = 4;                     // A buffers: step kt reads kt % 4 while kt + 1..3 arrive
template <int BM> constexpr int threads_for() { return 64 * kWN * (BM / 64); }
// The epilogue stages the bf16 output tile in the first two A buffers (BM / 2
// rows each, rows of OS elements: padded by 8 at BM = 128, unpadded at 64 so
// that four workgroups fit a CU's LDS).
template <int BM, bool SWIGLU> constexpr int out_stride() { return (SWIGLU ? kBN / 2 : kBN) + (BM == 128 ? 8 : 0); }
template <int BM, bool SWIGLU> constexpr int abuf01_bytes() {
    return BM * 128 > BM / 2 * out_stride<BM, SWIGLU>() * 2 ? BM * 128 : BM / 2 * out_stride<BM, SWIGLU>() * 2;
}

// A rows sit in LDS unpadded, the 16-byte chunk q of tile row r at physical
// chunk q ^ a_swz(r), a_swz(r) = (r / 2) % 8.  Measured on MI355X for the
// MFMA operand reads (lane l reads row l % 32 at logical chunk 2 s + l / 32,
// ds_read_b128): 1.00 against 1.12 for rows padded to 144 bytes, 1.8 for the
// XORs r % 8 and (r + r / 8) % 8, and 7.0 unswizzled.
__host__ __device__ constexpr int a_swz(int r) { return (r >> 1) & 7; }

// Wait until at most N vector memory operations of this wave are outstanding
// and its LDS operations are done, then the workgroup barrier.  One asm
// statement with a memory clobber: no memory operation moves across it, and
// unlike __syncthreads it does not wait for every outstanding load.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
    static_assert(N >= 0 && N <= 63, "vmcnt holds 0..63");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

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
    int gs;            // group stride on the padded K axis, ceil_to(group, 64)
    int kpad;          // padded K; the last group ends here
    int half_n;        // SWIGLU: N / 2 (gate column n pairs with up column n + half_n)
    int tpg;           // GMODE 3: K steps per group stride
    int tiles_m, tiles_n, band;
    uint32_t a_bytes, w_bytes, s_bytes;
    bool vec_out;      // y 16-byte aligned with ldy % 8 == 0: 16-byte output stores
    int bm;            // tile rows: 128 or 64
    bool cols;         // group stride 128 at 128 rows: 128 x 32 wave tiles (gemm_prefill_cols_kernel)
    int splits;        // gemm_prefill_cols_kernel: workgroups along K (blockIdx.y); > 1 writes fp32 sums to R
    float* R;          // splits > 1: fp32 sums before the token scale [splits, M, ldr]
    int64_t ldr;       // NB * 16
    // The reference's mid-group tensors (gemm_prefill_kernel with CM > 0): A
    // holds the activation bytes compat_act_kernel rebuilt from the two
    // planes, W the packed codes [N, kb] and S the weight scales [G, N] as
    // stored, c_as the activation scales as fp32 [G, M] (rebuilt), c_ak the
    // ksums [G, ld_as] and c_wz the zero points [G, N] (CM == 2) as stored.
    const float* c_as;
    const int32_t* c_ak;
    const uint16_t* c_wz;
    int ld_as, kb;
    uint32_t as_bytes, ak_bytes;
    bool cwt;          // compat W in launch_midgroup_tile's 1 KB tiles instead of rows as stored
};

constexpr uint32_t kOOB = 0x80000000u;   // an offset past every buffer here (all below 2^31 bytes)

// Workgroups are dispatched round-robin over the 8 XCDs, each with its own
// L2.  Renumber them so that every XCD walks one contiguous run of tiles, and
// order the tiles in bands of p.band tile rows, so the workgroups resident on
// one XCD at a time cover a compact block of the output and share A rows and
// weight columns in that XCD's L2.
__device__ __forceinline__ void tile_of(const PrefillParams& p, int& tile_m, int& tile_n) {
    const int nwg = static_cast<int>(gridDim.x);
    const int bid = static_cast<int>(blockIdx.x);
    const int xcd = bid & 7, q = nwg >> 3, r = nwg & 7;
    const int lin = xcd * q + min(xcd, r) + (bid >> 3);
    const int band = lin / (p.band * p.tiles_n);
    const int inband = lin - band * p.band * p.tiles_n;
    const int rows = min(p.band, p.tiles_m - band * p.band);
    tile_m = band * p.band + inband % rows;
    tile_n = inband / rows;
}

// The bf16 output tile, staged in LDS as BM rows of OC columns (row stride OS
// elements; rows 0..BM/2-1 from lo, the rest from hi), leaves as 16-byte row
// stores of 8 columns per thread and step; rows past M are skipped, and a
// chunk past the last column (or a row that cannot take 16-byte stores) is
// stored element by element.
template <int BM, int THREADS, int OC, int OS>
__device__ __forceinline__ void store_tile(const PrefillParams& p, const uint16_t* lo, const uint16_t* hi, int m0,
                                           int n0, int ncols, int tid) {
    constexpr int CPR = OC / 8;   // chunks per row
#pragma unroll
    for (int k = 0; k < BM * CPR / THREADS; ++k) {
        const int c = tid + k * THREADS;
        const int r = c / CPR, c8 = (c % CPR) * 8;
        const int row = m0 + r, col = n0 + c8;
        if (row >= p.M || col >= ncols) continue;
        const uint4 v = *reinterpret_cast<const uint4*>((r < BM / 2 ? lo : hi) + (r % (BM / 2)) * OS + c8);
        uint16_t* y = p.Y + static_cast<int64_t>(row) * p.ldy + col;
        if (p.vec_out && col + 8 <= ncols) {
            *reinterpret_cast<uint4*>(y) = v;
        } else {
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 8; ++q)
                if (col + q < ncols) y[q] = static_cast<uint16_t>(w[q >> 1] >> (16 * (q & 1)));
        }
    }
}

// K is walked in the padded group layout (kgeom.h): group g starts at g*gs,
// only the last group may be shorter, and it ends at kpad.
// GMODE: 0 = stride 64 (two groups per step), 1 = stride 128 (one per step),
// 3 = stride 128*t, t >= 2 (a group spans t steps and ends on a step's last
// slab, or on the last step), 2 = any other stride (groups may start and end
// on either 64-K half).
// SWIGLU: a wave's two 32-column blocks are 32 gate columns and the matching
// up columns, so each lane holds both operands of its outputs
// silu(y[:, n]) * y[:, n + N/2] (a tile covers 64 outputs); every column
// accumulates exactly as in the plain GEMM.
// CM: the reference's mid-group compat GEMM (1 symmetric, 2 with zero
// points; group stride 128*t, t >= 2), y = bf16(sum_g (float(I_g) * ws) * as)
// with I_g = P_g + wz * a_ksum, the fold order of ReferenceMidGroupGemm
// (int4_cube_lab/host/gemm_ref.cpp:199-240).  WT: the weights repacked into
// tiles per call (as the per-token path's, natural K order; the activation
// rows rebuilt in natural order).  Otherwise they are read as stored: lane
// (column c, half hh) takes bytes 32 hh .. 32 hh + 31 of its column's 64-byte
// step, so slab s holds codes 64 hh + 16 s + [0, 16) in unpack order (even
// codes, then odd, per dword), and compat_act_kernel writes each activation
// row's bytes in that same K order at the positions the operand reads below
// take (logical chunk 2 s + hh).  The per-row activation
// scales and ksums of a group reach LDS through a four-step register ring (one
// dword load per lane and step: rows 0..BM-1 of the scales by the first BM
// threads, of the ksums by the others), written a step before the group's
// fold reads them.
template <int GMODE, int DW, bool SBF16, bool DUMP, bool SWIGLU, int BM, int CM = 0, bool WT = false>
__global__ __launch_bounds__(threads_for<BM>(), 2) void gemm_prefill_kernel(const PrefillParams p) {
    constexpr int kThreads = threads_for<BM>();
    constexpr int kBM = BM;
    constexpr int kABuf = BM * 128;              // one step's A tile in LDS (unpadded 128-byte rows)
    constexpr int kABuf01 = abuf01_bytes<BM, SWIGLU>();
    constexpr bool COMPAT = CM > 0;
    constexpr bool RAWW = COMPAT && !WT;   // compat weights read as stored (else repacked tiles)
    static_assert(kNA == BM * 8 / kThreads, "four 16-byte A chunks per lane per step");
    static_assert(!(SWIGLU && DUMP), "the SwiGLU variant dumps nothing");
    static_assert(!COMPAT || (GMODE == 3 && !DUMP && !SWIGLU && SBF16 && kThreads == 2 * BM),
                  "the compat variant: group stride 128*t (t >= 2), bf16 scales, no dump, no SwiGLU");
    // Four separate A buffers (separate objects, so the compiler's tracking of
    // loads into LDS keeps reads of one buffer from waiting on loads into
    // another).
    __shared__ __attribute__((aligned(16))) int8_t la0[kABuf01];
    __shared__ __attribute__((aligned(16))) int8_t la1[kABuf01];
    __shared__ __attribute__((aligned(16))) int8_t la2[kABuf];
    __shared__ __attribute__((aligned(16))) int8_t la3[kABuf];
    // buffer b (a compile-time index after unrolling)
    auto abuf = [&](int b) -> int8_t* { return b == 0 ? la0 : (b == 1 ? la1 : (b == 2 ? la2 : la3)); };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / kWN;  // 0..BM / 64 - 1
    const int wn = wave % kWN;
    int tile_m, tile_n;
    tile_of(p, tile_m, tile_n);
    const int m0 = tile_m * kBM;
    const int n0 = tile_n * (SWIGLU ? kBN / 2 : kBN);
    const int c32 = lane & 31;   // column (B) / row (A) inside a 32-block
    const int hh = lane >> 5;    // K half of the 32-K slab

    const auto ra_rsrc = make_rsrc(p.A, p.a_bytes);
    const auto rw_rsrc = make_rsrc(p.W, p.w_bytes);
    const auto rs_rsrc = make_rsrc(p.S, p.s_bytes);

    // Token scales of the tile's rows: requested now, parked in LDS for the
    // epilogue (a load issued there would add a memory round trip per row).
    __shared__ uint32_t tsl[kBM];
    uint32_t ts_bits = 0;
    if constexpr (!COMPAT) {
        if (tid < kBM && m0 + tid < p.M) ts_bits = p.a_scale[m0 + tid];
    }

    // ---- weights: byte offsets of this lane's two 16-byte chunks per step,
    // for the wave's 32-column blocks j = 0, 1 (column blocks past N read 0).
    // Compat: chunk 0 holds slabs 0-1 and chunk 1 slabs 2-3 of the stored
    // row; columns past N read zero.
    uint32_t woff[2][2];
    uint32_t soff[2];
    int colj[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int col = SWIGLU ? n0 + wn * 32 + c32 + j * p.half_n : n0 + wn * 64 + j * 32 + c32;
        colj[j] = col;
        if constexpr (RAWW) {
            // the column's step bytes 32 hh .. +31: quads 2 hh and 2 hh + 1 of a
            // compat tile (256 bytes apart), or 32 contiguous bytes of its row
            const bool in = col < p.N;
            if (p.cwt) {
                woff[j][0] = in ? static_cast<uint32_t>(col >> 4) * static_cast<uint32_t>(p.KT) * 1024u +
                                      (32u * hh + static_cast<uint32_t>(col & 15)) * 16u
                                : kOOB;
                woff[j][1] = woff[j][0] + 256u;
            } else {
                woff[j][0] = in ? static_cast<uint32_t>(col) * static_cast<uint32_t>(p.kb) + 32u * hh : kOOB;
                woff[j][1] = woff[j][0] + 16u;
            }
        } else {
            const uint32_t tile0 = static_cast<uint32_t>(col >> 4) * static_cast<uint32_t>(p.KT) * 1024u;
            woff[j][0] = tile0 + static_cast<uint32_t>((col & 15) + 16 * hh) * 16u;        // slabs 0, 2
            woff[j][1] = tile0 + static_cast<uint32_t>((col & 15) + 16 * (2 + hh)) * 16u;  // slabs 1, 3
        }
        if constexpr (COMPAT) soff[j] = col < p.N ? static_cast<uint32_t>(col) * 2u : kOOB;
        else soff[j] = (static_cast<uint32_t>(col >> 4) * static_cast<uint32_t>(p.NG) * 16u + (col & 15)) * 2u;
    }

    // ---- activations: each step's A[128 rows][128 K] goes straight from
    // memory into an LDS buffer (16-byte buffer loads to LDS: lane l of a
    // load writes bytes 16 l..16 l + 15 of a contiguous 1 KB).  Load i of
    // wave w fills tile rows 32 w + 8 i..+8; lane l takes row + l / 8,
    // physical chunk l % 8, i.e. logical chunk (l % 8) ^ a_swz(row).
    uint32_t aoffg[kNA];
#pragma unroll
    for (int i = 0; i < kNA; ++i) {
        const int r = 8 * (kNA * wave + i) + (lane >> 3);
        const int q = (lane & 7) ^ a_swz(r);
        // rows >= M lie past the buffer and read zero; they are never stored
        aoffg[i] = static_cast<uint32_t>(m0 + r) * static_cast<uint32_t>(p.lda) + static_cast<uint32_t>(q) * 16u;
    }
    auto load_a = [&](int kt, int b) {
        // the padding half of a last step reads past kpad: zero weights there
        const uint32_t k = static_cast<uint32_t>(min(kt, p.KT - 1)) * 128u;
        int8_t* const dst = abuf(b) + kNA * 1024 * wave;
#pragma unroll
        for (int i = 0; i < kNA; ++i)
            buf_load16_lds(ra_rsrc, dst + 1024 * i, aoffg[i] + k);
    };

    uint4 wr[DW][2][2];
    auto load_w = [&](int slot, int kt) {
        const uint32_t t = static_cast<uint32_t>(min(kt, p.KT - 1)) * (RAWW && !p.cwt ? 64u : 1024u);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            wr[slot][j][0] = buf_load16(rw_rsrc, woff[j][0] + t);
            wr[slot][j][1] = buf_load16(rw_rsrc, woff[j][1] + t);
        }
    };
    // Scales of the groups that may end in step kt: at its 64-K halves h=0,1
    // (group 128 only ends on the step's last slab, so one scale suffices).
    constexpr bool ONE_END = GMODE == 1 || GMODE == 3;   // groups end only on a step's last slab
    // Group stride 128: each row block's fold is staggered against the other
    // row block's MFMAs (row block 1 folds during the next step).
    constexpr bool STAG = GMODE == 1;
    constexpr int NSC = ONE_END ? 1 : 2;
    auto load_s = [&](int kt, uint32_t (&sv)[2][NSC]) {
        const int ktc = min(kt, p.KT - 1);
#pragma unroll
        for (int h = 0; h < NSC; ++h) {
            const int g = min((ktc * 128 + (ONE_END ? 127 : h * 64 + 63)) / p.gs, p.NG - 1);
            const uint32_t go = static_cast<uint32_t>(g) * (COMPAT ? static_cast<uint32_t>(p.N) * 2u : 32u);
#pragma unroll
            for (int j = 0; j < 2; ++j) sv[j][h] = buf_load_u16(rs_rsrc, soff[j] + go);
        }
    };
    // Compat: the zero points of the same groups (CM == 2), and the row ring.
    // Vector memory operations per step: kNA A chunks, four weight chunks,
    // the scales (and zero points), the ring's dword.
    constexpr int kStepVm = kNA + 4 + 2 * NSC * (CM == 2 ? 2 : 1) + (COMPAT ? 1 : 0);
    const auto rz_rsrc = make_rsrc(p.c_wz, CM == 2 ? static_cast<uint32_t>(p.NG) * static_cast<uint32_t>(p.N) * 2u : 0u);
    auto load_z = [&](int kt, uint32_t (&zv)[2][NSC]) {
        if constexpr (CM == 2) {
            const int ktc = min(kt, p.KT - 1);
#pragma unroll
            for (int h = 0; h < NSC; ++h) {
                const int g = min((ktc * 128 + (ONE_END ? 127 : h * 64 + 63)) / p.gs, p.NG - 1);
                const uint32_t go = static_cast<uint32_t>(g) * static_cast<uint32_t>(p.N) * 2u;
#pragma unroll
                for (int j = 0; j < 2; ++j) zv[j][h] = buf_load_u16(rz_rsrc, soff[j] + go);
            }
        }
    };
    // Row values of group g(kt) = min(kt / tpg, NG - 1): thread t < BM loads
    // the fp32 activation scale of tile row t, thread BM + t its ksum (a
    // wave-uniform choice); rows past M read zero.  Two LDS slots by group
    // parity: the value of g(kt + 1) is written during step kt, after the
    // barrier that ended the fold of group g(kt) - 1 (the same slot), and before
    // the barrier ahead of g(kt + 1)'s fold.
    // One LDS object for both (slot b: scales at cfv[2 b BM + r], ksums at
    // cfv[2 b BM + BM + r]): a store that picks between two objects is not
    // told apart from the A buffers' loads to LDS, and the compiler then
    // waits for those loads before it.
    __shared__ __attribute__((aligned(16))) uint32_t cfv[COMPAT ? 4 * kBM : 1];
    const bool as_wave = wave < kBM / 64;
    const int rvr = as_wave ? tid : tid - kBM;
    const uint32_t rvo = (m0 + rvr < p.M) ? static_cast<uint32_t>(m0 + rvr) * 4u : kOOB;
    const auto ras_rsrc = make_rsrc(p.c_as, COMPAT ? p.as_bytes : 0u);
    const auto rak_rsrc = make_rsrc(p.c_ak, COMPAT ? p.ak_bytes : 0u);
    auto group_of = [&](int kt) { return min(kt / p.tpg, p.NG - 1); };
    auto load_rv = [&](int kt) -> uint32_t {
        const uint32_t g = static_cast<uint32_t>(group_of(kt));
        if (as_wave) return buf_load_u32(ras_rsrc, rvo + g * static_cast<uint32_t>(p.M) * 4u);
        return buf_load_u32(rak_rsrc, rvo + g * static_cast<uint32_t>(p.ld_as) * 4u);
    };
    auto store_rv = [&](int kt, uint32_t v) { cfv[(group_of(kt) & 1) * 2 * kBM + (as_wave ? 0 : kBM) + rvr] = v; };

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
    const v16i zero16 = {};

    // acc[rb] += float(P[rb]) * w_scale for row block rb of group g;
    // ws2[j] are the scale bits of the wave's column blocks j = 0, 1.
    // Compat: acc[rb] += (float(P/16 + wz * a_ksum) * ws) * as, rounded at
    // each operation (zs2: the zero-point bits; the rows' values from LDS).
    auto fold_cm = [&](int rb, int g, const uint32_t (&ws2)[2], const uint32_t (&zs2)[2])
        __attribute__((always_inline)) {
        // the reference's separate roundings: no multiply-add contraction
#pragma clang fp contract(off)
        const int b = (g & 1) * 2 * kBM;
        float ws[2];
        int wz[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            ws[j] = bf16_bits_to_f32(ws2[j]);
            wz[j] = CM == 2 ? static_cast<int>(bf16_bits_to_f32(zs2[j])) : 0;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r0 = wm * 64 + rb * 32 + q * 8 + hh * 4;   // rows r0..r0+3: i = 4 q .. 4 q + 3
            const uint4 as4 = *reinterpret_cast<const uint4*>(&cfv[b + r0]);
            const uint4 ak4 = *reinterpret_cast<const uint4*>(&cfv[b + kBM + r0]);
            const float as[4] = {__uint_as_float(as4.x), __uint_as_float(as4.y), __uint_as_float(as4.z),
                                 __uint_as_float(as4.w)};
            const int ak[4] = {static_cast<int>(ak4.x), static_cast<int>(ak4.y), static_cast<int>(ak4.z),
                               static_cast<int>(ak4.w)};
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int i = q * 4 + e;
                    const int I = (P[rb][j][i] >> 4) + (CM == 2 ? wz[j] * ak[e] : 0);
                    const float t1 = static_cast<float>(I) * ws[j];
                    acc[rb][j][i] = acc[rb][j][i] + t1 * as[e];
                }
        }
    };
    auto fold_rb = [&](int rb, int g, const uint32_t (&ws2)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float ws = scale_to_f32<SBF16>(ws2[j]);
            if constexpr (DUMP) {
                const int col = colj[j];
                if (g >= 0 && g < p.NG) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int row = m0 + wm * 64 + rb * 32 + (i >> 2) * 8 + hh * 4 + (i & 3);
                        if (row < p.M && col < p.N)
                            p.P[(static_cast<int64_t>(g) * p.M + row) * p.N + col] = P[rb][j][i] >> 4;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[rb][j][i] += static_cast<float>(P[rb][j][i]) * ws;
        }
    };

    // ---- prologue: A(0..2) to their LDS buffers, then W(0..DW-1) and the
    // first scales (the empty asm statements keep this issue order, which the
    // wait below counts on)
    // Compat: group 0's row values first (written to LDS below), the ring's
    // next three entries after the scales.
    uint32_t rv[4] = {0u, 0u, 0u, 0u};
    uint32_t rv0 = 0u;
    if constexpr (COMPAT) rv0 = load_rv(0);
    load_a(0, 0);
    load_a(1, 1);
    load_a(2, 2);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int s = 0; s < DW; ++s) load_w(s, s);
    uint32_t sc[2][NSC];
    load_s(0, sc);
    uint32_t zc[2][NSC] = {};
    load_z(0, zc);
    if constexpr (COMPAT) {
        rv[1] = load_rv(1);
        rv[2] = load_rv(2);
        rv[3] = load_rv(3);
    }
    asm volatile("" ::: "memory");
    // STAG: the scale bits of the previous step's groups (zero before step 0,
    // whose fold of row block 1 adds zero partials times zero)
    uint32_t scp[2] = {0u, 0u};
    if (tid < kBM) tsl[tid] = ts_bits;
    if constexpr (COMPAT) store_rv(0, rv0);
    // A(0) has landed once at most the loads issued after it are outstanding
    // (A(1), A(2), the weight ring, the scales, the row ring); then every
    // wave's part of it is in LDS
    wait_vm_barrier<2 * kNA + DW * 4 + (kStepVm - kNA - 4) + (COMPAT ? 2 : 0)>();

    // This lane's A operand offsets for slab s of row block 0 (row block 1 is
    // 32 rows = 4096 bytes further): row wm * 64 + c32, logical chunk 2 s + hh.
    uint32_t aread[4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
        aread[s] = static_cast<uint32_t>((wm * 64 + c32) * 128 + (((2 * s + hh) ^ a_swz(c32)) * 16));

    // Per step: issue the loads for later steps, unpack this step's weights
    // into all four slabs' B operands (so the ring slot is dead and its refill
    // needs no register copies), then the MFMAs.
    auto step = [&](int kt, int u, int buf) __attribute__((always_inline)) {
        // A(kt + 3) into the buffer step kt - 1 read
        load_a(kt + 3, (buf + 3) % kNB);
        uint32_t scn[2][NSC];
        load_s(kt + 1, scn);
        uint32_t zcn[2][NSC] = {};
        load_z(kt + 1, zcn);
        if constexpr (COMPAT) {
            // ring entry of step kt - 3 (landed: the barrier ending step kt - 1
            // waited for it) -> LDS; this step's entry is group g(kt + 4)'s
            store_rv(kt + 1, rv[(buf + 1) & 3]);
            rv[buf] = load_rv(kt + 4);
        }
        // A operands from LDS two slabs at a time: slabs 0-1 now (their
        // latency hides behind the weight unpack), slabs 2-3 before slab 1's
        // MFMAs.  The scheduling barrier keeps the first reads ahead of the
        // unpack; reading slab by slab right before each MFMA pair exposes
        // the LDS latency eight times per step.  Group stride 64 (a fold in
        // mid-step) and the partial dump need those registers and read per
        // slab.
        constexpr bool PAIRS = GMODE != 0 && !DUMP && !STAG;
        const int8_t* ab = abuf(buf);
        auto lds_a = [&](int rb, int s) { return *reinterpret_cast<const v4i*>(ab + aread[s] + rb * 4096); };
        v4i avs[4][2];
        if constexpr (STAG) {
            // row block 0's A operands now (their latency hides behind the
            // unpack), row block 1's at the start of row block 0's MFMAs
#pragma unroll
            for (int s = 0; s < 4; ++s) avs[s][0] = lds_a(0, s);
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (PAIRS) {
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) avs[s][rb] = lds_a(rb, s);
            __builtin_amdgcn_sched_barrier(0);
        }
        v4i bvs[4][2];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                // repacked: chunk s % 2, half s / 2; stored compat rows:
                // chunk s / 2, half s % 2
                const uint4 w = wr[u][j][RAWW ? (s >> 1) : (s & 1)];
                const bool upper = RAWW ? (s & 1) : (s >> 1);
                const uint32_t d0 = upper ? w.z : w.x;
                const uint32_t d1 = upper ? w.w : w.y;
                bvs[s][j] = v4i{unpack_lo4(d0), unpack_hi4(d0), unpack_lo4(d1), unpack_hi4(d1)};
            }
        load_w(u, kt + DW);

        if constexpr (STAG) {
            // Group stride 128 (a group per step): row block 0's eight MFMAs,
            // with the previous step's row block 1 folded in between them, then
            // row block 1's, with this step's row block 0 folded in between.
            // Each half step pairs 8 MFMAs (256 cycles of the matrix core)
            // with 64 fold instructions (256 VALU cycles) of independent
            // registers, so one wave keeps both pipes busy; the group's first
            // slab takes a zero accumulator operand.
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                if (rb == 0) {
#pragma unroll
                    for (int s = 0; s < 4; ++s) avs[s][1] = lds_a(1, s);
                }
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int j = 0; j < 2; ++j) P[rb][j] = mfma32(avs[s][rb], bvs[s][j], s == 0 ? zero16 : P[rb][j]);
                if (rb == 0) {
                    fold_rb(1, kt - 1, scp);
                } else {
                    const uint32_t ws2[2] = {sc[0][0], sc[1][0]};
                    fold_rb(0, kt, ws2);
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);   // eight VALU
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                scp[j] = sc[j][0];
                sc[j][0] = scn[j][0];
            }
            return;
        }

        // Slab-major: the four blocks' MFMA chains interleave, so no MFMA waits
        // on its predecessor's result.  A group ends after slab 1 or 3 (fixed
        // for strides 64/128, one uniform test per step for 128*t, per half
        // otherwise); both row blocks are folded then.  Strides 64/128 start
        // each group with a zero accumulator operand; the others, whose group
        // starts are not known at compile time, clear the accumulators after a
        // fold (a per-MFMA select would cost 16 VALU operations per MFMA).
        // Groups past NG (the padding half of a last step) hold zero partials
        // and fold nothing; a short last group that ends on the lower half
        // folds after the upper half's zero weights.
        bool step_ends = false;
        if constexpr (GMODE == 3) step_ends = (kt + 1) % p.tpg == 0 || kt == p.KT - 1;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const bool fresh = GMODE == 0 ? (s == 0 || s == 2) : (GMODE == 1 && s == 0);
            if (PAIRS && s == 1) {
#pragma unroll
                for (int s2 = 2; s2 < 4; ++s2)
#pragma unroll
                    for (int rb = 0; rb < 2; ++rb) avs[s2][rb] = lds_a(rb, s2);
            }
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                const v4i av = PAIRS ? avs[s][rb] : lds_a(rb, s);
#pragma unroll
                for (int j = 0; j < 2; ++j) P[rb][j] = mfma32(av, bvs[s][j], fresh ? zero16 : P[rb][j]);
            }
            if (s == 1 || s == 3) {
                const int kend = kt * 128 + (s + 1) * 32;   // K position after this slab
                const int g = (kend - 1) / p.gs;
                bool ends;
                if constexpr (GMODE == 0) ends = true;
                else if constexpr (GMODE == 1) ends = s == 3;
                else if constexpr (GMODE == 3) ends = s == 3 && step_ends;
                else ends = kend <= p.kpad && (kend % p.gs == 0 || kend == p.kpad);
                if (ends) {
                    const int h = ONE_END ? 0 : (s >> 1);
                    const uint32_t ws2[2] = {sc[0][h], sc[1][h]};
                    if constexpr (COMPAT) {
                        const uint32_t zs2[2] = {zc[0][h], zc[1][h]};
                        fold_cm(0, g, ws2, zs2);
                        fold_cm(1, g, ws2, zs2);
                    } else {
                        fold_rb(0, g, ws2);
                        fold_rb(1, g, ws2);
                    }
                    if constexpr (GMODE >= 2) {
#pragma unroll
                        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                            for (int j = 0; j < 2; ++j) P[rb][j] = zero16;
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int h = 0; h < NSC; ++h) {
                sc[j][h] = scn[j][h];
                zc[j][h] = zcn[j][h];
            }
    };

    // Steps are unrolled by kNB (a multiple of DW), so the A buffer and the
    // weight ring slot of each step are compile-time indices.  A step issues
    // exactly kStepVm vector memory operations (the partial dump
    // only adds stores, which make the wait below stricter); A(kt + 1), loaded
    // during step kt - 2, has landed once at most the two newest steps'
    // operations are outstanding, and after the barrier every wave's part of
    // it is in LDS.  The barrier also ends every read of the buffer step kt + 1
    // refills.
    static_assert(kNB % DW == 0, "an unrolled group covers whole weight rings");
    auto one = [&](int kt, int u) __attribute__((always_inline)) {
        step(kt, u % DW, u % kNB);
        wait_vm_barrier<2 * kStepVm>();
    };
    // Whole groups of kNB steps, then the remaining steps after the loop: an
    // early exit inside the unrolled group would give the loop header a path
    // whose newest loads are this group's weight refills, and the wait counts
    // at the top of every iteration would have to cover it.
    int kt = 0;
    for (; kt + kNB <= p.KT; kt += kNB) {
#pragma unroll
        for (int u = 0; u < kNB; ++u) one(kt + u, u);
    }
#pragma unroll
    for (int u = 0; u < kNB - 1; ++u)
        if (kt + u < p.KT) one(kt + u, u);
    if constexpr (STAG) fold_rb(1, p.KT - 1, scp);   // the last step's row block 1

    // ---- epilogue: the tile's bf16 outputs go through LDS (the first two A
    // buffers, rows 0-63 and 64-127, are free once every load into LDS has
    // landed and every wave passed the barrier below) and leave as 16-byte
    // row stores.  Output tile: kBM rows x OC columns (OC = kBN, or kBN / 2
    // SwiGLU outputs), row stride OS elements.
    constexpr int OC = SWIGLU ? kBN / 2 : kBN;
    constexpr int OS = out_stride<BM, SWIGLU>();
    constexpr int RPA = BM / 2;   // output rows per staging buffer
    static_assert(RPA * OS * 2 <= kABuf01, "half the output rows fit an A buffer");
    wait_vm_barrier<0>();
    // rows 0..RPA-1 in la0, the rest in la1
    auto orow = [&](int r) -> uint16_t* {
        return reinterpret_cast<uint16_t*>(r < RPA ? la0 : la1) + (r % RPA) * OS;
    };
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = wm * 64 + rb * 32 + (i >> 2) * 8 + hh * 4 + (i & 3);   // row in the tile
            const float ts = COMPAT ? 1.0f : bf16_bits_to_f32(tsl[r]) * 0.0625f;
            if constexpr (SWIGLU) {
                orow(r)[wn * 32 + c32] =
                    static_cast<uint16_t>(swiglu_bf16_bits(acc[rb][0][i] * ts, acc[rb][1][i] * ts));
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    orow(r)[wn * 64 + j * 32 + c32] = static_cast<uint16_t>(f32_to_bf16_bits(acc[rb][j][i] * ts));
            }
        }
    }
    __syncthreads();
    store_tile<kBM, kThreads, OC, OS>(p, reinterpret_cast<const uint16_t*>(la0), reinterpret_cast<const uint16_t*>(la1),
                                      m0, n0, SWIGLU ? p.half_n : p.N, tid);
}

constexpr int kDW = 2;   // weight prefetch depth in K steps

// Group stride 128 without the partial dump or the SwiGLU pairs: the same
// BM x 128 tile (BM = 128 or 64) and K step, but each of the four waves owns
// all BM rows and one 32-column block (instead of 64 x 64 per wave; at 64
// rows, four waves per tile instead of two, three workgroups per CU).  Every weight is then loaded and
// unpacked by one wave instead of two: half the weight loads, and the unpack
// of each B operand serves four MFMAs instead of two (1.5 instead of 3 VALU
// instructions per MFMA; at 64 rows still 3), for twice the A operand reads
// from LDS.  Row block
// rb's fold runs during row block rb + 1's MFMAs (row block 3's during the next
// step's row block 0), one MFMA to eight fold instructions.  Each output's
// arithmetic is the 64 x 64 kernel's: outputs are bit-identical.
template <bool SBF16, int BM>
__global__ __launch_bounds__(256, BM == 64 ? 3 : 2) void gemm_prefill_cols_kernel(const PrefillParams p) {
    constexpr int kBM = BM, kThreads = 256;
    constexpr int RB = BM / 32;                  // 32-row blocks per wave
    constexpr int NA = BM * 8 / kThreads;        // 16-byte A chunks per lane per step
    constexpr int kABuf = kBM * 128;
    constexpr int kABuf01 = abuf01_bytes<BM, false>();
    static_assert(BM == 64 || BM == 128, "64- or 128-row tiles");
    __shared__ __attribute__((aligned(16))) int8_t la0[kABuf01];
    __shared__ __attribute__((aligned(16))) int8_t la1[kABuf01];
    __shared__ __attribute__((aligned(16))) int8_t la2[kABuf];
    __shared__ __attribute__((aligned(16))) int8_t la3[kABuf];
    auto abuf = [&](int b) -> int8_t* { return b == 0 ? la0 : (b == 1 ? la1 : (b == 2 ? la2 : la3)); };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // the wave's 32-column block
    int tile_m, tile_n;
    tile_of(p, tile_m, tile_n);
    const int m0 = tile_m * kBM;
    const int n0 = tile_n * kBN;
    const int c32 = lane & 31;
    const int hh = lane >> 5;
    // This workgroup's K steps [ka, ka + nk): the KT steps split evenly over
    // p.splits workgroups (the host keeps splits <= KT; one step is one group).
    const int ks = static_cast<int>(blockIdx.y);
    const int ka = (ks * p.KT) / p.splits;
    const int nk = ((ks + 1) * p.KT) / p.splits - ka;

    const auto ra_rsrc = make_rsrc(p.A, p.a_bytes);
    const auto rw_rsrc = make_rsrc(p.W, p.w_bytes);
    const auto rs_rsrc = make_rsrc(p.S, p.s_bytes);

    // token scales of the tile's rows, times the 1/16 of the unpack (exact),
    // as fp32 in LDS for the epilogue's 16-byte reads of four rows
    __shared__ __attribute__((aligned(16))) float tsl[kBM];
    uint32_t ts_bits = 0;
    if (tid < kBM && m0 + tid < p.M) ts_bits = p.a_scale[m0 + tid];

    // weights: this lane's two 16-byte chunks per step of the wave's block
    const int col = n0 + wave * 32 + c32;
    const uint32_t tile0 = static_cast<uint32_t>(col >> 4) * static_cast<uint32_t>(p.KT) * 1024u;
    const uint32_t woff0 = tile0 + static_cast<uint32_t>((col & 15) + 16 * hh) * 16u;        // slabs 0, 2
    const uint32_t woff1 = tile0 + static_cast<uint32_t>((col & 15) + 16 * (2 + hh)) * 16u;  // slabs 1, 3
    const uint32_t soff = (static_cast<uint32_t>(col >> 4) * static_cast<uint32_t>(p.NG) * 16u + (col & 15)) * 2u;

    // activations: as in gemm_prefill_kernel (wave w stages tile rows 8 NA w..+8 NA)
    uint32_t aoffg[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int r = 8 * (NA * wave + i) + (lane >> 3);
        const int q = (lane & 7) ^ a_swz(r);
        aoffg[i] = static_cast<uint32_t>(m0 + r) * static_cast<uint32_t>(p.lda) + static_cast<uint32_t>(q) * 16u;
    }
    auto load_a = [&](int kt, int b) {
        const uint32_t k = static_cast<uint32_t>(ka + min(kt, nk - 1)) * 128u;
        int8_t* const dst = abuf(b) + NA * 1024 * wave;
#pragma unroll
        for (int i = 0; i < NA; ++i)
            buf_load16_lds(ra_rsrc, dst + 1024 * i, aoffg[i] + k);
    };
    uint4 wr[kDW][2];
    auto load_w = [&](int slot, int kt) {
        const uint32_t t = static_cast<uint32_t>(ka + min(kt, nk - 1)) * 1024u;
        wr[slot][0] = buf_load16(rw_rsrc, woff0 + t);
        wr[slot][1] = buf_load16(rw_rsrc, woff1 + t);
    };
    // group stride 128: step kt is group kt (the padding half of a last step
    // meets zero weights)
    auto load_s = [&](int kt) -> uint32_t {
        const int g = min(ka + min(kt, nk - 1), p.NG - 1);
        return buf_load_u16(rs_rsrc, soff + static_cast<uint32_t>(g) * 32u);
    };

    v16i P[RB];
    float acc[RB][16];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            P[rb][i] = 0;
            acc[rb][i] = 0.0f;
        }
    const v16i zero16 = {};
    auto fold = [&](int rb, uint32_t wsb) __attribute__((always_inline)) {
        const float ws = scale_to_f32<SBF16>(wsb);
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[rb][i] += static_cast<float>(P[rb][i]) * ws;
    };

    // ---- prologue (the issue order the first wait counts on)
    load_a(0, 0);
    load_a(1, 1);
    load_a(2, 2);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int s = 0; s < kDW; ++s) load_w(s, s);
    uint32_t sc = load_s(0);
    asm volatile("" ::: "memory");
    uint32_t scp = 0u;   // the previous step's scale (the last row block folds one step late)
    if (tid < kBM) tsl[tid] = bf16_bits_to_f32(ts_bits) * 0.0625f;
    wait_vm_barrier<2 * NA + kDW * 2 + 1>();

    uint32_t aread[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) aread[s] = static_cast<uint32_t>(c32 * 128 + (((2 * s + hh) ^ a_swz(c32)) * 16));

    auto step = [&](int kt, int u, int buf) __attribute__((always_inline)) {
        load_a(kt + 3, (buf + 3) % kNB);
        const uint32_t scn = load_s(kt + 1);
        const int8_t* ab = abuf(buf);
        auto lds_a = [&](int rb, int s) { return *reinterpret_cast<const v4i*>(ab + aread[s] + rb * 4096); };
        v4i av[2][4];
#pragma unroll
        for (int s = 0; s < 4; ++s) av[0][s] = lds_a(0, s);
        __builtin_amdgcn_sched_barrier(0);
        v4i bvs[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint4 w = wr[u][s & 1];
            const uint32_t d0 = (s >> 1) ? w.z : w.x;
            const uint32_t d1 = (s >> 1) ? w.w : w.y;
            bvs[s] = v4i{unpack_lo4(d0), unpack_hi4(d0), unpack_lo4(d1), unpack_hi4(d1)};
        }
        load_w(u, kt + kDW);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            if (rb < RB - 1) {
#pragma unroll
                for (int s = 0; s < 4; ++s) av[(rb + 1) & 1][s] = lds_a(rb + 1, s);
            }
#pragma unroll
            for (int s = 0; s < 4; ++s) P[rb] = mfma32(av[rb & 1][s], bvs[s], s == 0 ? zero16 : P[rb]);
            if (rb == 0) fold(RB - 1, scp);
            else fold(rb - 1, sc);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);   // eight VALU
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        scp = sc;
        sc = scn;
    };
    // a step issues NA + 3 vector memory operations; the wait keeps the two
    // newest steps' in flight (A(kt + 1), issued in step kt - 2, has landed)
    auto one = [&](int kt, int u) __attribute__((always_inline)) {
        step(kt, u % kDW, u % kNB);
        wait_vm_barrier<2 * (NA + 3)>();
    };
    int kt = 0;
    for (; kt + kNB <= nk; kt += kNB) {
#pragma unroll
        for (int u = 0; u < kNB; ++u) one(kt + u, u);
    }
#pragma unroll
    for (int u = 0; u < kNB - 1; ++u)
        if (kt + u < nk) one(kt + u, u);
    fold(RB - 1, scp);   // the last step's last row block

    // ---- epilogue: as in gemm_prefill_kernel, through the first two A buffers
    constexpr int OC = kBN;
    constexpr int OS = out_stride<BM, false>();
    constexpr int RPA = kBM / 2;
    wait_vm_barrier<0>();   // also: no load into LDS outlives the workgroup
    if (p.splits > 1) {
        // this split's fp32 sums, before the token scale, for wide_reduce_kernel
        // (which adds the splits in index order, scales and rounds)
        const int col = n0 + wave * 32 + c32;
        if (col < p.N) {
            float* const r = p.R + static_cast<int64_t>(ks) * p.M * p.ldr + col;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int row = m0 + rb * 32 + (i >> 2) * 8 + hh * 4 + (i & 3);
                    if (row < p.M) r[static_cast<int64_t>(row) * p.ldr] = acc[rb][i];
                }
        }
        return;
    }
    auto orow = [&](int r) -> uint16_t* {
        return reinterpret_cast<uint16_t*>(r < RPA ? la0 : la1) + (r % RPA) * OS;
    };
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r0 = rb * 32 + q * 8 + hh * 4;   // this lane's four rows r0..r0+3
            const float4 ts = *reinterpret_cast<const float4*>(&tsl[r0]);
            const float tv[4] = {ts.x, ts.y, ts.z, ts.w};
#pragma unroll
            for (int j = 0; j < 4; j += 2) {
                const uint32_t v = f32x2_to_bf16x2_bits(acc[rb][q * 4 + j] * tv[j], acc[rb][q * 4 + j + 1] * tv[j + 1]);
                orow(r0 + j)[wave * 32 + c32] = static_cast<uint16_t>(v);
                orow(r0 + j + 1)[wave * 32 + c32] = static_cast<uint16_t>(v >> 16);
            }
        }
    __syncthreads();
    store_tile<kBM, kThreads, OC, OS>(p, reinterpret_cast<const uint16_t*>(la0), reinterpret_cast<const uint16_t*>(la1),
                                      m0, n0, p.N, tid);
}

// The reference's mid-group activation planes rebuilt for the compat variant
// of gemm_prefill_kernel: row `blockIdx.x` of A [Ma, KT * 128], whose 16-byte
// chunk L = 2 s + hh of step kt holds the codes kt * 128 + 64 hh + 16 s +
// [0, 16) (even codes of each dword first, as act_pair builds them; codes past
// kpad are zero), and the row's activation scales as fp32 into as32 [G, Ma].
// NAT: natural K order instead (chunk L of step kt: codes kt * 128 + 16 L +
// [0, 16), byte i = code i), for the repacked weight tiles.
template <bool NAT>
__global__ __launch_bounds__(256) void compat_act_kernel(const uint8_t* __restrict__ hi,
                                                         const uint8_t* __restrict__ lo,
                                                         const uint16_t* __restrict__ a_scale, int ld_as, int kb,
                                                         int kpad, int Ma, int KT, int NG, int8_t* __restrict__ A,
                                                         float* __restrict__ as32) {
    const int64_t row = blockIdx.x;
    const int ci = static_cast<int>(blockIdx.y) * 256 + static_cast<int>(threadIdx.x);
    if (ci < KT * 8) {
        const int L = ci & 7, kt = ci >> 3;
        const int k0 = NAT ? kt * 128 + 16 * L : kt * 128 + 64 * (L & 1) + 16 * (L >> 1);
        uint4 out = make_uint4(0u, 0u, 0u, 0u);
        if (k0 < kpad) {   // k0 and kpad are multiples of 16: the chunk is whole
            const int64_t src = row * kb + k0 / 2;
            const uint2 h = *reinterpret_cast<const uint2*>(hi + src);
            const uint2 l = *reinterpret_cast<const uint2*>(lo + src);
            int e0, o0, e1, o1;
            act_pair(h.x, l.x, e0, o0);
            act_pair(h.y, l.y, e1, o1);
            if (NAT) {
                // bytes [e.b0, o.b0, e.b1, o.b1], [e.b2, o.b2, e.b3, o.b3]
                const uint32_t ue0 = e0, uo0 = o0, ue1 = e1, uo1 = o1;
                out = make_uint4(__builtin_amdgcn_perm(uo0, ue0, 0x05010400u), __builtin_amdgcn_perm(uo0, ue0, 0x07030602u),
                                 __builtin_amdgcn_perm(uo1, ue1, 0x05010400u), __builtin_amdgcn_perm(uo1, ue1, 0x07030602u));
            } else {
                out = make_uint4(static_cast<uint32_t>(e0), static_cast<uint32_t>(o0), static_cast<uint32_t>(e1),
                                 static_cast<uint32_t>(o1));
            }
        }
        *reinterpret_cast<uint4*>(A + row * (static_cast<int64_t>(KT) * 128) + 16 * ci) = out;
    }
    if (blockIdx.y == 0)
        for (int g = static_cast<int>(threadIdx.x); g < NG; g += 256)
            as32[static_cast<int64_t>(g) * Ma + row] = bf16_bits_to_f32(a_scale[static_cast<int64_t>(g) * ld_as + row]);
}

template <int GMODE, bool SBF16, bool DUMP, bool SWIGLU>
hipError_t launch_g(const PrefillParams& p, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n));
    // The partial dump keeps 128-row tiles (the compiler fails on the 64-row
    // dump variants); each output element's arithmetic does not depend on the
    // tile height, so its outputs equal the 64-row kernel's bit for bit.
    if constexpr (GMODE == 1 && !DUMP && !SWIGLU) {
        if (p.cols) {
            if (p.bm == 128) gemm_prefill_cols_kernel<SBF16, 128><<<grid, dim3(256), 0, stream>>>(p);
            else gemm_prefill_cols_kernel<SBF16, 64><<<grid, dim3(256), 0, stream>>>(p);
            return hipGetLastError();
        }
    }
    if (p.bm == 64 && !DUMP)
        gemm_prefill_kernel<GMODE, kDW, SBF16, false, SWIGLU, 64><<<grid, dim3(threads_for<64>()), 0, stream>>>(p);
    else
        gemm_prefill_kernel<GMODE, kDW, SBF16, DUMP, SWIGLU, 128><<<grid, dim3(threads_for<128>()), 0, stream>>>(p);
    return hipGetLastError();
}

template <bool SBF16, bool DUMP, bool SWIGLU>
hipError_t launch(const PrefillParams& p, hipStream_t stream) {
    if (p.gs == 64) return launch_g<0, SBF16, DUMP, SWIGLU>(p, stream);
    if (p.gs == 128) return launch_g<1, SBF16, DUMP, SWIGLU>(p, stream);
    if (p.gs % 128 == 0) return launch_g<3, SBF16, DUMP, SWIGLU>(p, stream);
    return launch_g<2, SBF16, DUMP, SWIGLU>(p, stream);
}

}  // namespace

// The 128 x 32 wave tiles for group stride 128 (defined 0 only for
// side-by-side measurements of the 64 x 64 kernel).
#ifndef W4A8_PREFILL_COLS
#define W4A8_PREFILL_COLS 1
#endif

int64_t prefill_workspace_bytes(int64_t, int64_t, int64_t, int64_t) { return 0; }

// The compat GEMM on gemm_prefill_kernel (group stride 128 * t, t >= 2, more
// than kMidPrefillMinRows rows, and 64-row output tiles for at least half the
// CUs: with fewer, the mid-group kernel's K split over waves is faster -- on
// MI355X at 128 rows, qkv / o / down_proj 25.9 / 24.0 / 124 against 35.6 /
// 33.0 / 149 us, gate_up 145 against 86 us; from 256 rows this path wins on
// all four, 1.1-1.8x).  Wide N meets the tile rule from one row tile on:
// gate_up on weight tiles at 24 / 32 / 48 / 64 rows 43.6 / 43.8 / 45.3 / 46.6
// against 54.2 / 64.7 / 76.8 / 97.7 us on the mid-group kernel, at 16 rows
// 43.8 against 29.6 for its shared-activation kernel.  Workspace: the rebuilt activation rows,
// then the fp32 activation scales, then (from W4A8_MID_TILED_MIN_ROWS rows)
// the weight tiles repacked from w_q for this call, each 256-byte aligned.
// Reading w_q as stored, a wave's 16-byte loads cover 32 columns' half lines
// each, against one 1 KB tile for the repacked layout; the repack streams the
// weights once more (2 N kpad / 2 bytes), which the larger calls repay.  0
// where the shape takes the mid-group kernel (gemm_midgroup.hip) instead.
// Tiled against stored weights on MI355X, us (qkv / o / gate_up / down,
// repack included; bench graph replays): 1024 rows 67 / 62 / 450 / 288
// against 74 / 60 / 504 / 302; 4096 rows 218 / 158 / 1423 / 746 against 248 /
// 175 / 1646 / 805 (at 512 rows the stored weights were ahead).
#ifndef W4A8_MID_PREFILL_MIN_ROWS
#define W4A8_MID_PREFILL_MIN_ROWS 16
#endif
constexpr int64_t kMidPrefillMinRows = W4A8_MID_PREFILL_MIN_ROWS;
#ifndef W4A8_MID_TILED_MIN_ROWS
#define W4A8_MID_TILED_MIN_ROWS 1024
#endif

namespace {

struct MidPrefillLayout {
    int64_t a_off, as_off, wt_off, bytes;
    bool tiled;
};

MidPrefillLayout mid_prefill_layout(int64_t Ma, int64_t N, int64_t K, int64_t group, bool w_tiles = false) {
    MidPrefillLayout l{0, 0, 0, 0, false};
    const int64_t gs = geom::group_stride(group);
    if (Ma <= kMidPrefillMinRows || gs % 128 != 0 || gs < 256 || N <= 0 || K <= 0) return l;
    if (geom::ceil_div(Ma, int64_t{64}) * geom::ceil_div(N, int64_t{kBN}) * 2 < device_cu_count()) return l;
    const int64_t KT = geom::k_tiles(K, group), lda = KT * 128, kb = geom::kpad(K, group) / 2;
    const int64_t ng = geom::num_groups(K, group);
    const int64_t wt = geom::col_blocks(N) * KT * geom::kTileBytes;
    const int64_t lim = int64_t{1} << 31;
    // every buffer offset of the kernel, tile overhang included, below 2^31
    if ((Ma + 128) * lda >= lim || (N + 128) * kb >= lim || ng * (N + 128) * 2 >= lim || ng * Ma * 4 >= lim ||
        wt + 8 * geom::kTileBytes * KT >= lim)
        return l;
    l.tiled = !w_tiles && Ma >= W4A8_MID_TILED_MIN_ROWS;   // tiles given: read them, no repack
    l.a_off = 0;
    l.as_off = geom::ceil_to(Ma * lda, int64_t{256});
    l.wt_off = geom::ceil_to(l.as_off + ng * Ma * 4, int64_t{256});
    l.bytes = l.tiled ? l.wt_off + wt : l.as_off + ng * Ma * 4;
    return l;
}

template <bool WT>
void launch_mid_prefill(const PrefillParams& p, bool asym, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n));
    if (p.bm == 64) {
        if (asym) gemm_prefill_kernel<3, kDW, true, false, false, 64, 2, WT><<<grid, dim3(threads_for<64>()), 0, stream>>>(p);
        else gemm_prefill_kernel<3, kDW, true, false, false, 64, 1, WT><<<grid, dim3(threads_for<64>()), 0, stream>>>(p);
    } else {
        if (asym) gemm_prefill_kernel<3, kDW, true, false, false, 128, 2, WT><<<grid, dim3(threads_for<128>()), 0, stream>>>(p);
        else gemm_prefill_kernel<3, kDW, true, false, false, 128, 1, WT><<<grid, dim3(threads_for<128>()), 0, stream>>>(p);
    }
}

}  // namespace

int64_t midgroup_prefill_workspace_bytes(int64_t Ma, int64_t N, int64_t K, int64_t group) {
    return mid_prefill_layout(Ma, N, K, group).bytes;
}

hipError_t launch_gemm_midgroup_prefill(const MidgroupArgs& a, void* ws, int64_t ws_bytes, hipStream_t stream) {
    const MidPrefillLayout l = mid_prefill_layout(a.Ma, a.N, a.K, a.group, a.w_tiles);
    const int64_t ng = geom::num_groups(a.K, a.group);
    if (l.bytes == 0 || ws == nullptr || ws_bytes < l.bytes || a.partials != nullptr ||
        ng * a.ld_as * 4 >= (int64_t{1} << 31))
        return hipErrorInvalidValue;
    char* const w = static_cast<char*>(ws);
    const int64_t KT = geom::k_tiles(a.K, a.group), lda = KT * 128;
    PrefillParams p{};
    p.A = reinterpret_cast<const int8_t*>(w + l.a_off);
    p.lda = lda;
    p.c_as = reinterpret_cast<const float*>(w + l.as_off);
    p.c_ak = static_cast<const int32_t*>(a.a_ksum);
    p.c_wz = static_cast<const uint16_t*>(a.w_zero);
    p.ld_as = static_cast<int>(a.ld_as);
    p.kb = static_cast<int>(geom::kpad(a.K, a.group) / 2);
    p.W = l.tiled ? reinterpret_cast<const uint4*>(w + l.wt_off) : static_cast<const uint4*>(a.w_q);
    p.cwt = a.w_tiles;
    p.S = static_cast<const uint16_t*>(a.w_scale);
    p.Y = static_cast<uint16_t*>(a.y);
    p.ldy = a.ldy;
    p.M = static_cast<int>(a.Ma);
    p.N = static_cast<int>(a.N);
    p.K = static_cast<int>(a.K);
    p.KT = static_cast<int>(KT);
    p.NG = static_cast<int>(ng);
    p.NB = static_cast<int>(geom::col_blocks(a.N));
    p.gs = static_cast<int>(geom::group_stride(a.group));
    p.kpad = static_cast<int>(geom::kpad(a.K, a.group));
    p.tpg = p.gs / 128;
    p.bm = prefill_tile_rows(a.Ma, a.N, a.group, false);
    p.tiles_m = static_cast<int>(geom::ceil_div(a.Ma, int64_t{p.bm}));
    p.tiles_n = static_cast<int>(geom::ceil_div(a.N, int64_t{kBN}));
    p.band = 4;
    p.a_bytes = static_cast<uint32_t>(a.Ma * lda);
    p.w_bytes = static_cast<uint32_t>(l.tiled || a.w_tiles ? p.NB * KT * geom::kTileBytes : a.N * p.kb);
    p.s_bytes = static_cast<uint32_t>(ng * a.N * 2);
    p.as_bytes = static_cast<uint32_t>(ng * a.Ma * 4);
    p.ak_bytes = static_cast<uint32_t>(ng * a.ld_as * 4);
    p.vec_out = (reinterpret_cast<uintptr_t>(a.y) % 16 == 0) && (a.ldy % 8 == 0);
    p.splits = 1;
    const dim3 agrid(static_cast<unsigned>(a.Ma), static_cast<unsigned>(geom::ceil_div(KT * 8, int64_t{256})));
    const auto* hi = static_cast<const uint8_t*>(a.a_hi);
    const auto* lo = static_cast<const uint8_t*>(a.a_lo);
    const auto* as = static_cast<const uint16_t*>(a.a_scale);
    auto* A = reinterpret_cast<int8_t*>(w + l.a_off);
    auto* as32 = reinterpret_cast<float*>(w + l.as_off);
    if (l.tiled) {
        hipError_t e = launch_repack_weights(static_cast<const uint8_t*>(a.w_q), reinterpret_cast<uint8_t*>(w + l.wt_off),
                                             a.N, a.K, a.group, stream);
        if (e != hipSuccess) return e;
        compat_act_kernel<true><<<agrid, dim3(256), 0, stream>>>(hi, lo, as, p.ld_as, p.kb, p.kpad, p.M, p.KT, p.NG, A,
                                                                  as32);
    } else {
        compat_act_kernel<false><<<agrid, dim3(256), 0, stream>>>(hi, lo, as, p.ld_as, p.kb, p.kpad, p.M, p.KT, p.NG, A,
                                                                   as32);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (l.tiled) launch_mid_prefill<true>(p, a.w_zero != nullptr, stream);
    else launch_mid_prefill<false>(p, a.w_zero != nullptr, stream);
    return hipGetLastError();
}

int prefill_tile_rows(int64_t M, int64_t N, int64_t group, bool swiglu) {
    const int64_t tn = swiglu ? geom::ceil_div(N / 2, kBN / 2) : geom::ceil_div(N, kBN);
    const int64_t tiles = geom::ceil_div(M, int64_t{128}) * tn, cus = device_cu_count();
    if (W4A8_PREFILL_COLS && !swiglu && geom::group_stride(group) == 128) {
        // The four-wave tiles of gemm_prefill_cols_kernel (64-row tiles run
        // three workgroups per CU, 128-row tiles two).  64 rows up to 1.5
        // tiles of 128 rows per CU and between 2 and 4 per CU; 128 rows where
        // they fill the CUs about once (up to 2 per CU) or many times.
        // Measured on MI355X at the QwQ-32B shapes (64 / 128 rows, us): o_proj
        // M=1024 37.0 / 41.7, M=2048 63.3 / 66.2, M=4096 123.1 / 116.5; qkv
        // M=256 17.8 / 25.3, M=1024 49.1 / 45.1, M=4096 171 / 165; down M=1024
        // 179 / 198; gate_up M=256 86 / 88, M=512 167 / 156.
        return (tiles * 2 <= cus * 3 || (tiles > 2 * cus && tiles <= 4 * cus)) ? 64 : 128;
    }
    // The 64 x 64 wave tiles (other group strides, SwiGLU): 64-row tiles
    // (twice as many, up to four workgroups per CU) where the 128-row ones
    // would leave CUs idle or unevenly loaded: at most one for every second
    // CU, or between one and two per CU.  Measured on MI355X (QwQ-32B shapes,
    // 128 -> 64 rows): o_proj M=1024 49.2 -> 46.1 us, down_proj M=1024 222 ->
    // 205 us, qkv/o/down M=128-256 3-6% faster; at M=512 (at most one
    // 128-row tile per CU) 64 rows lose 30-50%.
    return (tiles <= cus / 2 || (tiles > cus && tiles <= 2 * cus)) ? 64 : 128;
}

hipError_t launch_gemm_prefill(const GemmArgs& a, hipStream_t stream) {
    return launch_gemm_prefill_bm(a, prefill_tile_rows(a.M, a.N, a.group, a.swiglu), stream);
}

// Decode-sized row counts (up to 64) on narrow N: one 64-row tile of the
// 128 x 32 wave kernel spans few workgroups (40 on o_proj), so K is split
// over `splits` workgroups (group stride 128: every step is one group) and
// wide_reduce_kernel adds the fp32 split sums in index order, scales by the
// token scale and rounds -- the same reduction as the wide kernel's K split.
int64_t prefill_split_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group, int splits) {
    const int64_t s = std::min<int64_t>(splits, geom::k_tiles(K, group));
    return s > 1 ? s * M * geom::col_blocks(N) * 16 * 4 : 0;
}

hipError_t launch_gemm_prefill_split(const GemmArgs& a, int splits, hipStream_t stream) {
    if (a.swiglu || a.partials || geom::group_stride(a.group) != 128 || a.M <= 0 || a.M > 64 || splits < 1)
        return hipErrorInvalidValue;
    const int64_t need = prefill_split_workspace_bytes(a.M, a.N, a.K, a.group, splits);
    if (need > 0 && (a.workspace == nullptr || a.workspace_bytes < need)) return hipErrorInvalidValue;
    PrefillParams p{};
    p.A = a.a_q;
    p.lda = a.lda;
    p.a_scale = a.a_scale;
    p.W = reinterpret_cast<const uint4*>(a.w_tiles);
    p.S = a.s_tiles;
    p.Y = a.y;
    p.ldy = a.ldy;
    p.M = static_cast<int>(a.M);
    p.N = static_cast<int>(a.N);
    p.K = static_cast<int>(a.K);
    p.KT = static_cast<int>(geom::k_tiles(a.K, a.group));
    p.NG = static_cast<int>(geom::num_groups(a.K, a.group));
    p.NB = static_cast<int>(geom::col_blocks(a.N));
    p.gs = 128;
    p.kpad = static_cast<int>(geom::kpad(a.K, a.group));
    p.tpg = 1;
    p.bm = 64;
    p.tiles_m = 1;
    p.tiles_n = static_cast<int>(geom::ceil_div(a.N, kBN));
    p.band = 4;
    p.a_bytes = static_cast<uint32_t>((a.M - 1) * a.lda + p.kpad);
    p.w_bytes = static_cast<uint32_t>(geom::col_blocks(a.N) * geom::k_tiles(a.K, a.group) * geom::kTileBytes);
    p.s_bytes = static_cast<uint32_t>(geom::col_blocks(a.N) * geom::num_groups(a.K, a.group) * 16 * 2);
    p.vec_out = (reinterpret_cast<uintptr_t>(a.y) % 16 == 0) && (a.ldy % 8 == 0);
    p.cols = true;
    p.splits = need > 0 ? static_cast<int>(std::min<int64_t>(splits, p.KT)) : 1;
    p.R = static_cast<float*>(a.workspace);
    p.ldr = static_cast<int64_t>(p.NB) * 16;
    const dim3 grid(static_cast<unsigned>(p.tiles_n), static_cast<unsigned>(p.splits));
    if (a.scale_bf16) gemm_prefill_cols_kernel<true, 64><<<grid, dim3(256), 0, stream>>>(p);
    else gemm_prefill_cols_kernel<false, 64><<<grid, dim3(256), 0, stream>>>(p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.splits == 1) return e;
    return launch_split_reduce(p.R, p.ldr, p.a_scale, p.Y, p.ldy, p.M, p.N, p.splits, false, a.scale_bf16, p.S,
                               nullptr, stream);
}

hipError_t launch_gemm_prefill_bm(const GemmArgs& a, int bm, hipStream_t stream) {
    if (bm != 64 && bm != 128) return hipErrorInvalidValue;
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
    p.gs = static_cast<int>(geom::group_stride(a.group));
    p.kpad = static_cast<int>(geom::kpad(a.K, a.group));
    p.tpg = p.gs / 128;
    p.bm = a.partials ? 128 : bm;
    bm = p.bm;
    p.tiles_m = static_cast<int>(geom::ceil_div(a.M, p.bm));
    p.half_n = a.swiglu ? static_cast<int>(a.N / 2) : 0;
    p.tiles_n = static_cast<int>(a.swiglu ? geom::ceil_div(a.N / 2, kBN / 2) : geom::ceil_div(a.N, kBN));
    p.band = 4;
    // rows end at kpad; the padding half of a last step meets zero weights and
    // in the last row reads out of range (zero)
    p.a_bytes = static_cast<uint32_t>((a.M - 1) * a.lda + p.kpad);
    p.w_bytes = static_cast<uint32_t>(geom::col_blocks(a.N) * geom::k_tiles(a.K, a.group) * geom::kTileBytes);
    p.s_bytes = static_cast<uint32_t>(geom::col_blocks(a.N) * geom::num_groups(a.K, a.group) * 16 * 2);
    p.vec_out = (reinterpret_cast<uintptr_t>(a.y) % 16 == 0) && (a.ldy % 8 == 0);
    p.cols = W4A8_PREFILL_COLS != 0;
    p.splits = 1;
    if (a.swiglu) return a.scale_bf16 ? launch<true, false, true>(p, stream) : launch<false, false, true>(p, stream);
    const bool dump = a.partials != nullptr;
    if (a.scale_bf16) return dump ? launch<true, true, false>(p, stream) : launch<true, false, false>(p, stream);
    return dump ? launch<false, true, false>(p, stream) : launch<false, false, false>(p, stream);
}

}  // namespace w4a8
