// Grouped-query attention over the decoder's KV cache (gfx950, bf16 MFMA).
//
// The query heads that share a KV head are the rows of one attention problem:
// for sequence b and KV head h the rows are r = t * G + g (query token t, head
// h * G + g of that token), and row r attends to the cache positions
// 0 .. p(r), p(r) = pos[0] + t clamped to [0, L) (causal; the current token's
// own key and value were appended by w4a8_rope_kv before this call).
//
// Cache layouts (one axis of Lc positions per (b, h), Lc a multiple of 64):
//   K  [B, KVH, Lc, D]  a key is 2 D contiguous bytes
//   Vt [B, KVH, D, Lc]  V transposed: one value dimension is contiguous over positions
// so that every MFMA operand a lane needs is one contiguous 16-byte read.
//
// Arithmetic of a row, in chunks of 64 positions:
//   scores  S^T = K . Q^T by v_mfma_f32_16x16x32_bf16 (keys as the A rows, the
//           16 query rows of a tile as the B columns) in fp32, times
//           c = log2(e) * scale; positions past p(r) are -inf;
//   chunk   flash update of the running state (m, l, O) of the split the
//           chunk belongs to: m' = max(m, max_k s), alpha = 2^(m - m'),
//           P = 2^(s - m'), l' = l * alpha + sum_k P, O' = O * alpha +
//           bf16(P) . V (MFMA: V^T as the A rows, P^T as the B columns);
//   splits  `cps` consecutive chunks form a split; split states are combined
//           in the order s = 0, 1, ... by (m1, l1, O1) (+) (m2, l2, O2) =
//           (m, l1 a1 + l2 a2, O1 a1 + O2 a2), m = max(m1, m2), a_i = 2^(m_i - m);
//   output  bf16(O * (1 / l)).
// Every sum runs in an order that does not depend on which other rows share
// a tile, so a row's result depends only on its query, the cache and cps: the
// decode launch (one single-wave workgroup per split, the chunk operands
// loaded straight into registers one chunk ahead, split states through a
// workspace, then a combine kernel) and the prefill launch (four waves share
// each chunk through LDS and walk every split of their rows) return the same
// bits for the same row.  Float contraction is off in this file; each fused
// multiply-add is written out.
#include <math.h>

#include <algorithm>

#include "common.h"
#include "launch.h"

namespace w4a8 {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;        // cache positions per chunk (four 16-key MFMA tiles)
constexpr int kStateHead = 4;     // floats before O in a workspace state: m, l, 2 unused

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Chunk-relative position of S^T row c of key tile kt, and of the score lane
// group j holds at slot e of that tile.  Tiles 2s and 2s + 1 together hold
// positions 32s .. 32s + 31, lane group j eight consecutive ones (32s + 8j ..
// +8, four from each tile): the P^T operand of key block s and the 16-byte
// V^T read of lane group j then cover the same eight positions.
__device__ __forceinline__ int tile_row_pos(int kt, int c) {
    return 32 * (kt >> 1) + 8 * (c >> 2) + 4 * (kt & 1) + (c & 3);
}
__device__ __forceinline__ int lane_pos(int kt, int j, int e) { return 32 * (kt >> 1) + 8 * j + 4 * (kt & 1) + e; }

// A operands of one chunk: K for the score MFMAs (tile kt, k-step i: lane (c, j)
// holds key tile_row_pos(kt, c), dims 32 i + 8 j .. +8) and V^T for the output
// MFMAs (dim tile dt, key block s: lane (c, j) holds dim 16 dt + c at positions
// 32 s + 8 j .. +8).
template <int D>
struct KOps {
    uint4 k[4][D / 32];
};
template <int D>
struct VOps {
    uint4 v[D / 16][2];
};

// Running state of one query row.  The row's four lanes (c, j = 0..3) each
// hold m and l and the slice O^T[16 dt + 4 j + e][c], e = 0..3, of its O.
template <int D>
struct RowState {
    float m, l;
    f32x4 o[D / 16];
};

template <int D>
__device__ __forceinline__ void state_clear(RowState<D>& s) {
    s.m = -INFINITY;
    s.l = 0.0f;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) s.o[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
}

// The split combine (+): coefficients from the two maxima, then every value
// as x1 * a1 + x2 * a2 with one rounding of the product x2 * a2 and a fused
// multiply-add.  Shared by the prefill kernel and the combine kernel.
__device__ __forceinline__ void fold_coeffs(float m1, float m2, float& mn, float& a1, float& a2) {
#pragma clang fp contract(off)
    mn = fmaxf(m1, m2);
    a1 = exp2f(m1 - mn);
    a2 = exp2f(m2 - mn);
}

__device__ __forceinline__ float fold_value(float x1, float a1, float x2, float a2) {
#pragma clang fp contract(off)
    return fmaf(x1, a1, x2 * a2);
}

// s = s (+) t; an empty state (l == 0: no position of the row in that split) is
// the identity.
template <int D>
__device__ __forceinline__ void state_fold(RowState<D>& s, const RowState<D>& t) {
#pragma clang fp contract(off)
    if (t.l == 0.0f) return;
    if (s.l == 0.0f) {
        s = t;
        return;
    }
    float mn, a1, a2;
    fold_coeffs(s.m, t.m, mn, a1, a2);
    s.l = fold_value(s.l, a1, t.l, a2);
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
        for (int e = 0; e < 4; ++e) s.o[dt][e] = fold_value(s.o[dt][e], a1, t.o[dt][e], a2);
    s.m = mn;
}

__device__ __forceinline__ int clamp_pos(int64_t p, int L) {
    return static_cast<int>(p < 0 ? 0 : (p >= L ? L - 1 : p));
}

// A 16-row tile of one (sequence, KV head) pair, seen from lane (c, j).
struct Tile {
    int pair;              // b * KVH + h
    int r;                 // this lane's row (c-th of the tile)
    bool real;             // r < G * T
    int tok;               // query token of row r
    int64_t q_off;         // element offset of row r in q and out
};

template <int D>
__device__ __forceinline__ Tile make_tile(const AttnArgs& a, int pair, int rt, int c) {
    Tile t;
    t.pair = pair;
    const int R = a.G * a.T;
    t.r = rt * 16 + c;
    t.real = t.r < R;
    t.tok = t.real ? t.r / a.G : 0;
    const int g = t.real ? t.r - t.tok * a.G : 0;
    const int b = pair / a.KVH, h = pair - b * a.KVH;
    t.q_off = ((static_cast<int64_t>(b) * a.T + t.tok) * a.H + h * a.G + g) * D;
    return t;
}

// The last position attended to by the real rows r0 .. r1 (r1 clamped to the problem).
__device__ __forceinline__ int last_pos(const AttnArgs& a, int64_t pos0, int r1) {
    return clamp_pos(pos0 + min(r1, a.G * a.T - 1) / a.G, a.L);
}

// Q^T as the B operand of the score MFMAs: lane (c, j) holds q[r][32 i + 8 j .. +8]
// for k-step i; rows past the problem read zero.
template <int D>
__device__ __forceinline__ void load_q(const AttnArgs& a, const Tile& t, int j, bf16x8 (&qop)[D / 32]) {
    const uint16_t* qr = a.q + t.q_off;
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
        const uint4 v = t.real ? *reinterpret_cast<const uint4*>(qr + 32 * i + 8 * j) : make_uint4(0, 0, 0, 0);
        qop[i] = __builtin_bit_cast(bf16x8, v);
    }
}

// The operands of the chunk at position c0 straight from memory.  `skip` (2^31)
// moves every offset past the buffer: the loads then read zero without touching
// memory, so a prefetch that is not needed costs no traffic and the loads stay
// unconditional (straight-line code keeps the compiler's waits counting only
// the older chunk).
constexpr uint32_t kSkip = 0x80000000u;

template <int D>
__device__ __forceinline__ void load_chunk_global(KOps<D>& ko, VOps<D>& vo, __amdgpu_buffer_rsrc_t kr,
                                                  __amdgpu_buffer_rsrc_t vr, int Lc, int c0, int c, int j,
                                                  uint32_t skip) {
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < D / 32; ++i)
            ko.k[kt][i] = buf_load16(
                kr, static_cast<uint32_t>(((c0 + tile_row_pos(kt, c)) * D + 32 * i + 8 * j) * 2) + skip);
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
        for (int s = 0; s < 2; ++s)
            vo.v[dt][s] =
                buf_load16(vr, static_cast<uint32_t>(((16 * dt + c) * Lc + c0 + 32 * s + 8 * j) * 2) + skip);
}

// Scores of one chunk: lane (c, j) gets S^T[lane_pos(kt, j, e)][row c].
template <int D>
__device__ __forceinline__ void chunk_scores(f32x4 (&sc)[4], const bf16x8 (&qop)[D / 32], const KOps<D>& ko) {
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
        sc[kt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < D / 32; ++i) sc[kt] = mfma_bf16(__builtin_bit_cast(bf16x8, ko.k[kt][i]), qop[i], sc[kt]);
    }
}

// The softmax update and the output product of one chunk (positions c0 ..).
template <int D>
__device__ __forceinline__ void chunk_update(RowState<D>& st, const f32x4 (&sc)[4], const VOps<D>& vo, int c0,
                                             int p_row, float cs, int j) {
#pragma clang fp contract(off)
    float x[4][4];
    float mloc = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[kt][e] = c0 + lane_pos(kt, j, e) <= p_row ? sc[kt][e] * cs : -INFINITY;
            mloc = fmaxf(mloc, x[kt][e]);
        }
    float mc = fmaxf(mloc, __shfl_xor(mloc, 16));
    mc = fmaxf(mc, __shfl_xor(mc, 32));
    const float mn = fmaxf(st.m, mc);
    const float mz = mn == -INFINITY ? 0.0f : mn;   // no position of the row yet: everything stays 0
    const float alpha = exp2f(st.m - mz);
    float p[4][4];
    float lsum = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            p[kt][e] = exp2f(x[kt][e] - mz);
            lsum = lsum + p[kt][e];
        }
    lsum = lsum + __shfl_xor(lsum, 16);
    lsum = lsum + __shfl_xor(lsum, 32);
    st.l = fmaf(st.l, alpha, lsum);
    st.m = mn;
    // P^T as the B operand of key block s: slots 0..7 = positions 32 s + 8 j + 0..7
    bf16x8 pop[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const uint4 w = make_uint4(f32x2_to_bf16x2_bits(p[2 * s][0], p[2 * s][1]),
                                   f32x2_to_bf16x2_bits(p[2 * s][2], p[2 * s][3]),
                                   f32x2_to_bf16x2_bits(p[2 * s + 1][0], p[2 * s + 1][1]),
                                   f32x2_to_bf16x2_bits(p[2 * s + 1][2], p[2 * s + 1][3]));
        pop[s] = __builtin_bit_cast(bf16x8, w);
    }
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
#pragma unroll
        for (int e = 0; e < 4; ++e) st.o[dt][e] = st.o[dt][e] * alpha;
#pragma unroll
        for (int s = 0; s < 2; ++s) st.o[dt] = mfma_bf16(__builtin_bit_cast(bf16x8, vo.v[dt][s]), pop[s], st.o[dt]);
    }
}

// bf16(O * (1 / l)) of the lane's slice of row r.
template <int D>
__device__ __forceinline__ void write_out(const AttnArgs& a, const Tile& t, const RowState<D>& st, int j) {
#pragma clang fp contract(off)
    if (!t.real) return;
    const float inv = 1.0f / st.l;
    uint16_t* o = a.out + t.q_off;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
        const uint2 w = make_uint2(f32x2_to_bf16x2_bits(st.o[dt][0] * inv, st.o[dt][1] * inv),
                                   f32x2_to_bf16x2_bits(st.o[dt][2] * inv, st.o[dt][3] * inv));
        *reinterpret_cast<uint2*>(o + 16 * dt + 4 * j) = w;
    }
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t pair_rsrc(const uint16_t* base, int pair, int Lc, int D) {
    const int64_t n = static_cast<int64_t>(Lc) * D;
    return make_rsrc(base + pair * n, static_cast<uint32_t>(n * 2));
}

// ---- decode with the rotary embedding and the KV-cache append fused in ----
// x (+ bias, rounded as a bf16 add), as w4a8_rope_kv reads an input element.
__device__ __forceinline__ float rope_in(uint32_t xbits, uint32_t bbits, bool has_bias) {
#pragma clang fp contract(off)
    const float v = bf16_bits_to_f32(xbits);
    return has_bias ? bf16_bits_to_f32(f32_to_bf16_bits(v + bf16_bits_to_f32(bbits))) : v;
}

// The elements 32 i + 8 j .. +8 (i < D/32) of head `hd` of one row (16-byte loads).
template <int D>
__device__ __forceinline__ void rope_load(const uint16_t* row, int hd, int j, uint4 (&x)[D / 32]) {
#pragma unroll
    for (int i = 0; i < D / 32; ++i) x[i] = *reinterpret_cast<const uint4*>(row + hd * D + 32 * i + 8 * j);
}

// The angle-table entries of the lane's pair indices 32 i + 8 j .. +8, i < D/64.
template <int D>
__device__ __forceinline__ void rope_angles(const float* row, int j, float4 (&t)[D / 64][2]) {
#pragma unroll
    for (int i = 0; i < D / 64; ++i) {
        t[i][0] = *reinterpret_cast<const float4*>(row + 32 * i + 8 * j);
        t[i][1] = *reinterpret_cast<const float4*>(row + 32 * i + 8 * j + 4);
    }
}

// Rotate-half of the lane's elements as w4a8_rope_kv computes them: for pair index
// d < D/2 (x1 = x[d], x2 = x[d + D/2], c = cos[p, d], s = sin[p, d]) y[d] = bf16(fl(x1 c)
// - fl(x2 s)), y[d + D/2] = bf16(fl(x2 c) + fl(x1 s)), no fused multiply-add.  Lane group
// j holds elements 32 i + 8 j + e; the partner of i < D/64 is i + D/64, in the same lane.
// Everything is in registers (x, the bias elements bx, the angle entries).
template <int D>
__device__ __forceinline__ void rope_rotate(const uint4 (&x)[D / 32], const uint4 (&bx)[D / 32], bool has_bias,
                                            const float4 (&cs)[D / 64][2], const float4 (&sn)[D / 64][2],
                                            uint4 (&y)[D / 32]) {
#pragma clang fp contract(off)
    constexpr int HI = D / 64;
#pragma unroll
    for (int i = 0; i < HI; ++i) {
        const uint32_t x1w[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
        const uint32_t x2w[4] = {x[i + HI].x, x[i + HI].y, x[i + HI].z, x[i + HI].w};
        const uint32_t b1w[4] = {bx[i].x, bx[i].y, bx[i].z, bx[i].w};
        const uint32_t b2w[4] = {bx[i + HI].x, bx[i + HI].y, bx[i + HI].z, bx[i + HI].w};
        const float cv[8] = {cs[i][0].x, cs[i][0].y, cs[i][0].z, cs[i][0].w, cs[i][1].x, cs[i][1].y, cs[i][1].z,
                             cs[i][1].w};
        const float sv[8] = {sn[i][0].x, sn[i][0].y, sn[i][0].z, sn[i][0].w, sn[i][1].x, sn[i][1].y, sn[i][1].z,
                             sn[i][1].w};
        uint32_t o1[4], o2[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            float r1[2], r2[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float x1 = rope_in(h ? (x1w[w] >> 16) : (x1w[w] & 0xffffu), h ? (b1w[w] >> 16) : (b1w[w] & 0xffffu),
                                         has_bias);
                const float x2 = rope_in(h ? (x2w[w] >> 16) : (x2w[w] & 0xffffu), h ? (b2w[w] >> 16) : (b2w[w] & 0xffffu),
                                         has_bias);
                const float c = cv[2 * w + h], sn1 = sv[2 * w + h];
                r1[h] = x1 * c - x2 * sn1;
                r2[h] = x2 * c + x1 * sn1;
            }
            o1[w] = f32x2_to_bf16x2_bits(r1[0], r1[1]);
            o2[w] = f32x2_to_bf16x2_bits(r2[0], r2[1]);
        }
        y[i] = make_uint4(o1[0], o1[1], o1[2], o1[3]);
        y[i + HI] = make_uint4(o2[0], o2[1], o2[2], o2[3]);
    }
}

// One bf16 of a 16-byte operand replaced (slot e of 8).
__device__ __forceinline__ uint4 put_bf16(uint4 v, int e, uint32_t bits) {
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t lo = (e == 2 * k) ? bits : (w[k] & 0xffffu);
        const uint32_t hi = (e == 2 * k + 1) ? bits : (w[k] >> 16);
        w[k] = lo | (hi << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// Decode launch: workgroup (split, row tile, pair) folds the chunks of its split,
// each chunk's operands requested while the previous one is computed.  With one
// split it writes the output; otherwise its state goes to the workspace (m, l,
// then O) for attn_combine_kernel.  ROPE (one query token per sequence): the
// query rows are rotated here from the qkv projection output, and the workgroup
// whose chunk holds the step's position puts the step's rotated k and raw v into
// its operands in place of the cache's (row tile 0 also writes them to the
// caches), so that the separate w4a8_rope_kv launch is not needed; the values
// are the bits w4a8_rope_kv would have written.
template <int D, bool ROPE>
__global__ __launch_bounds__(64) void attn_split_kernel(const AttnArgs a) {
    const int lane = static_cast<int>(threadIdx.x);
    const int c = lane & 15, j = lane >> 4;
    const int split = static_cast<int>(blockIdx.x), rt = static_cast<int>(blockIdx.y);
    const int nch = a.Lc / kChunk;
    const int first = split * a.cps, last = min(first + a.cps, nch);
    const Tile t = make_tile<D>(a, static_cast<int>(blockIdx.z), rt, c);
    const __amdgpu_buffer_rsrc_t kr = pair_rsrc(a.k, t.pair, a.Lc, D);
    const __amdgpu_buffer_rsrc_t vr = pair_rsrc(a.vt, t.pair, a.Lc, D);
    // the split's first chunk and the queries are requested before the position is known
    KOps<D> ka, kb;
    VOps<D> va, vb;
    load_chunk_global<D>(ka, va, kr, vr, a.Lc, first * kChunk, c, j, 0u);
    bf16x8 qop[D / 32];
    const int b = t.pair / a.KVH, h = t.pair - b * a.KVH;
    const int qhead = h * a.G + rt * 16 + c;                 // T = 1: row r = g
    const int khead = a.H + h, vhead = a.H + a.KVH + h;
    // ROPE: the query row, the step's k head and v elements (16 dt + c) and their bias
    // elements, all requested with the first chunk
    uint4 xq[D / 32], xk[D / 32], bq[D / 32], bk[D / 32];
    uint32_t xv[D / 16], bv[D / 16];
    const bool has_bias = ROPE && a.bias != nullptr;
    if constexpr (ROPE) {
        const uint16_t* row = a.qkv + static_cast<int64_t>(b) * a.ldq;
#pragma unroll
        for (int i = 0; i < D / 32; ++i) xq[i] = bq[i] = bk[i] = make_uint4(0, 0, 0, 0);
        if (t.real) rope_load<D>(row, qhead, j, xq);
        rope_load<D>(row, khead, j, xk);
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) xv[dt] = row[vhead * D + 16 * dt + c];
        if (has_bias) {
            if (t.real) rope_load<D>(a.bias, qhead, j, bq);
            rope_load<D>(a.bias, khead, j, bk);
#pragma unroll
            for (int dt = 0; dt < D / 16; ++dt) bv[dt] = a.bias[vhead * D + 16 * dt + c];
        }
    } else {
        load_q<D>(a, t, j, qop);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int64_t pos0 = a.pos[0];
    const int p_row = clamp_pos(pos0 + t.tok, a.L);
    const int p_max = last_pos(a, pos0, rt * 16 + 15);
    // ROPE: the step's position (inside the cache, else nothing is written and q is zero,
    // as w4a8_rope_kv does), the rotated q rows, and the step's rotated k / v (+ bias)
    const bool inside = ROPE && pos0 >= 0 && pos0 < a.L;
    uint4 knew[D / 32];
    uint32_t vnew[D / 16];
    if constexpr (ROPE) {
        float4 cs[D / 64][2], sn[D / 64][2];
        rope_angles<D>(a.cos + (inside ? pos0 : 0) * a.ldc, j, cs);
        rope_angles<D>(a.sin + (inside ? pos0 : 0) * a.ldc, j, sn);
        uint4 yq[D / 32];
        rope_rotate<D>(xq, bq, has_bias, cs, sn, yq);
        rope_rotate<D>(xk, bk, has_bias, cs, sn, knew);
#pragma unroll
        for (int i = 0; i < D / 32; ++i)
            qop[i] = __builtin_bit_cast(bf16x8, (inside && t.real) ? yq[i] : make_uint4(0, 0, 0, 0));
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt)
            vnew[dt] = has_bias ? f32_to_bf16_bits(rope_in(xv[dt], bv[dt], true)) : xv[dt];
    }
    if (first * kChunk > p_max) {                    // no position of the split is attended by the tile
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }
    // the chunk holding the step's position: its operand slots for that position
    const int pch = inside ? static_cast<int>(pos0) / kChunk : -1;
    const int pp = static_cast<int>(pos0) & (kChunk - 1);
    auto inject = [&](KOps<D>& ko, VOps<D>& vo) __attribute__((always_inline)) {
        const int kt_p = 2 * (pp >> 5) + ((pp & 7) >> 2), c_p = 4 * ((pp & 31) >> 3) + (pp & 3);
        const int s_p = pp >> 5, j_p = (pp & 31) >> 3, e_p = pp & 7;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int i = 0; i < D / 32; ++i)
                if (kt == kt_p && c == c_p) ko.k[kt][i] = knew[i];
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
            for (int s = 0; s < 2; ++s)
                if (s == s_p && j == j_p) vo.v[dt][s] = put_bf16(vo.v[dt][s], e_p, vnew[dt]);
        if (rt == 0) {                               // one workgroup per pair appends the step's k and v
            const int64_t n = static_cast<int64_t>(a.Lc) * D;
            if (c == c_p) {
#pragma unroll
                for (int i = 0; i < D / 32; ++i)
                    *reinterpret_cast<uint4*>(a.kw + t.pair * n + pos0 * D + 32 * i + 8 * j) = knew[i];
            }
            if (j == j_p) {
#pragma unroll
                for (int dt = 0; dt < D / 16; ++dt)
                    a.vtw[t.pair * n + static_cast<int64_t>(16 * dt + c) * a.Lc + pos0] = static_cast<uint16_t>(vnew[dt]);
            }
        }
    };
    RowState<D> st;
    state_clear(st);
    f32x4 sc[4];
    for (int ch = first;;) {
        const bool more = ch + 1 < last && (ch + 1) * kChunk <= p_max;
        load_chunk_global<D>(kb, vb, kr, vr, a.Lc, (ch + 1) * kChunk, c, j, more ? 0u : kSkip);
        __builtin_amdgcn_sched_barrier(0);
        if (ROPE && ch == pch) inject(ka, va);
        chunk_scores<D>(sc, qop, ka);
        chunk_update<D>(st, sc, va, ch * kChunk, p_row, a.cs, j);
        if (!more) break;
        ++ch;
        const bool more2 = ch + 1 < last && (ch + 1) * kChunk <= p_max;
        load_chunk_global<D>(ka, va, kr, vr, a.Lc, (ch + 1) * kChunk, c, j, more2 ? 0u : kSkip);
        __builtin_amdgcn_sched_barrier(0);
        if (ROPE && ch == pch) inject(kb, vb);
        chunk_scores<D>(sc, qop, kb);
        chunk_update<D>(st, sc, vb, ch * kChunk, p_row, a.cs, j);
        if (!more2) break;
        ++ch;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the skipped prefetch
    if (a.ns == 1) {
        write_out<D>(a, t, st, j);
        return;
    }
    if (!t.real) return;
    const int64_t R = static_cast<int64_t>(a.G) * a.T;
    float* w = a.ws + ((t.pair * R + t.r) * a.ns + split) * (D + kStateHead);
    if (j == 0) *reinterpret_cast<float2*>(w) = make_float2(st.m, st.l);
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) *reinterpret_cast<f32x4*>(w + kStateHead + 16 * dt + 4 * j) = st.o[dt];
}

// The split states of one row (workgroup pair * R + r), combined in split order.
// Lane l owns O values l * D/64 .. +D/64 (the slices the split kernel wrote).
// States are requested kBatch at a time before any is folded, the first batch
// before the position is read (states past the row's last split are not used).
constexpr int kBatch = 16;

template <int D>
__global__ __launch_bounds__(64) void attn_combine_kernel(const AttnArgs a) {
#pragma clang fp contract(off)
    constexpr int V = D / 64;
    const int lane = static_cast<int>(threadIdx.x);
    const int64_t R = static_cast<int64_t>(a.G) * a.T;
    const int64_t pr = blockIdx.x;
    const int pair = static_cast<int>(pr / R);
    const int r = static_cast<int>(pr - pair * R);
    const int tok = r / a.G, g = r - tok * a.G;
    const int b = pair / a.KVH, h = pair - b * a.KVH;
    const float* w0 = a.ws + pr * a.ns * (D + kStateHead);
    float M = -INFINITY, Ls = 0.0f, O[V];
#pragma unroll
    for (int v = 0; v < V; ++v) O[v] = 0.0f;
    int nsp = a.ns;                                  // lowered to the row's splits after the first batch is requested
    for (int s0 = 0; s0 < nsp; s0 += kBatch) {
        float m2[kBatch], l2[kBatch], o2[kBatch][V];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int s = min(s0 + u, a.ns - 1);
            const float* w = w0 + s * (D + kStateHead);
            m2[u] = w[0];
            l2[u] = w[1];
#pragma unroll
            for (int v = 0; v < V; ++v) o2[u][v] = w[kStateHead + lane * V + v];
        }
        if (s0 == 0) {
            const int p_row = clamp_pos(a.pos[0] + tok, a.L);
            nsp = p_row / (a.cps * kChunk) + 1;      // splits holding positions <= p_row
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            if (s0 + u >= nsp || l2[u] == 0.0f) continue;
            if (Ls == 0.0f) {
                M = m2[u];
                Ls = l2[u];
#pragma unroll
                for (int v = 0; v < V; ++v) O[v] = o2[u][v];
                continue;
            }
            float mn, a1, a2;
            fold_coeffs(M, m2[u], mn, a1, a2);
            Ls = fold_value(Ls, a1, l2[u], a2);
#pragma unroll
            for (int v = 0; v < V; ++v) O[v] = fold_value(O[v], a1, o2[u][v], a2);
            M = mn;
        }
    }
    const float inv = 1.0f / Ls;
    uint16_t* o = a.out + ((static_cast<int64_t>(b) * a.T + tok) * a.H + h * a.G + g) * D + lane * V;
    if constexpr (V == 2) {
        *reinterpret_cast<uint32_t*>(o) = f32x2_to_bf16x2_bits(O[0] * inv, O[1] * inv);
    } else {
        *o = static_cast<uint16_t>(f32_to_bf16_bits(O[0] * inv));
    }
}

// Prefill launch: a workgroup of four waves takes 64 rows (four 16-row tiles)
// of one pair and walks the chunks up to its last row's position; each chunk's
// K and V^T (32 KB at D = 128) go from memory straight into one of two LDS
// buffers, one chunk ahead, and every wave reads its operands from there.  Rows
// of 2D (K) or 128 (V^T) bytes are stored with their 16-byte chunks permuted
// (chunk q of row r at q ^ kswz(r) / q ^ vswz(r)) so that the operand reads of
// eight consecutive lanes fall in distinct banks.  Workgroups are numbered so
// that each XCD (workgroups go to the eight XCDs round-robin) takes a
// contiguous run -- the row groups of a few pairs, whose K and V stay in that
// XCD's L2 -- the row groups with the most positions first within each pair.
constexpr int kLoopWaves = 4;

template <int D>
__device__ __forceinline__ int kswz(int r) {
    return D == 128 ? (r & 15) : ((r >> 1) & 7);
}
__device__ __forceinline__ int vswz(int d) { return (d >> 1) & 7; }

template <int D>
__global__ __launch_bounds__(64 * kLoopWaves) void attn_loop_kernel(const AttnArgs a, int groups) {
    constexpr int KB = kChunk * D * 2;               // K bytes of a chunk
    constexpr int CB = 2 * KB;                       // K + V^T bytes of a chunk
    constexpr int LPT = CB / (64 * kLoopWaves * 16); // 16-byte loads per thread per chunk
    constexpr int KLD = KB / (64 * kLoopWaves * 16); // ... of which K
    // two chunk buffers as two arrays (the loop is unrolled by two), so the compiler
    // sees that the loads into one never alias the operand reads from the other
    __shared__ __attribute__((aligned(16))) char lds0[CB];
    __shared__ __attribute__((aligned(16))) char lds1[CB];
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid >> 6, lane = tid & 63;
    const int c = lane & 15, j = lane >> 4;
    const int nwg = static_cast<int>(gridDim.x), bid = static_cast<int>(blockIdx.x);
    const int xcd = bid & 7, q8 = nwg >> 3, rem = nwg & 7;
    const int lin = xcd * q8 + min(xcd, rem) + (bid >> 3);
    const int pair = lin / groups;
    const int grp = groups - 1 - (lin - pair * groups);
    const Tile t = make_tile<D>(a, pair, kLoopWaves * grp + wave, c);
    const __amdgpu_buffer_rsrc_t kr = pair_rsrc(a.k, t.pair, a.Lc, D);
    const __amdgpu_buffer_rsrc_t vr = pair_rsrc(a.vt, t.pair, a.Lc, D);
    // this thread's loads: load n lands at LDS byte n * 4096 + 16 * tid of the buffer
    uint32_t goff[LPT];
#pragma unroll
    for (int n = 0; n < LPT; ++n) {
        const int P = n * 64 * kLoopWaves * 16 + 16 * tid;
        if (n < KLD) {
            const int r = P / (2 * D), pq = (P % (2 * D)) / 16;
            goff[n] = static_cast<uint32_t>(r * 2 * D + 16 * (pq ^ kswz<D>(r)));
        } else {
            const int P2 = P - KB;
            const int d = P2 / 128, pq = (P2 % 128) / 16;
            goff[n] = static_cast<uint32_t>(d * a.Lc * 2 + 16 * (pq ^ vswz(d)));
        }
    }
    // chunk ch into buf; a chunk past the last one reads zero (kSkip) without memory traffic
    auto load_chunk = [&](int ch, char* buf, bool real) {
        char* dst = buf + 1024 * wave;
        const uint32_t skip = real ? 0u : kSkip;
#pragma unroll
        for (int n = 0; n < LPT; ++n) {
            if (n < KLD)
                buf_load16_lds(kr, dst + n * 4096, static_cast<uint32_t>(ch * kChunk * 2 * D) + goff[n] + skip);
            else
                buf_load16_lds(vr, dst + n * 4096, static_cast<uint32_t>(ch * kChunk * 2) + goff[n] + skip);
        }
    };
    load_chunk(0, lds0, true);
    bf16x8 qop[D / 32];
    load_q<D>(a, t, j, qop);
    const int64_t pos0 = a.pos[0];
    const int p_row = clamp_pos(pos0 + t.tok, a.L);
    const int nchunks = last_pos(a, pos0, kLoopWaves * 16 * grp + kLoopWaves * 16 - 1) / kChunk + 1;
    // this lane's operand addresses inside a chunk buffer
    uint32_t kaddr[4][D / 32], vaddr[D / 16][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < D / 32; ++i) {
            const int r = tile_row_pos(kt, c);
            kaddr[kt][i] = static_cast<uint32_t>(r * 2 * D + 16 * ((4 * i + j) ^ kswz<D>(r)));
        }
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int d = 16 * dt + c;
            vaddr[dt][s] = static_cast<uint32_t>(KB + d * 128 + 16 * ((4 * s + j) ^ vswz(d)));
        }
    RowState<D> tot, st;
    state_clear(tot);
    state_clear(st);
    auto step = [&](const char* buf, int ch) {
        KOps<D> ko;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int i = 0; i < D / 32; ++i) ko.k[kt][i] = *reinterpret_cast<const uint4*>(buf + kaddr[kt][i]);
        f32x4 sc[4];
        chunk_scores<D>(sc, qop, ko);
        VOps<D> vo;
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
            for (int s = 0; s < 2; ++s) vo.v[dt][s] = *reinterpret_cast<const uint4*>(buf + vaddr[dt][s]);
        chunk_update<D>(st, sc, vo, ch * kChunk, p_row, a.cs, j);
        if ((ch + 1) % a.cps == 0 || ch + 1 == nchunks) {
            state_fold<D>(tot, st);
            state_clear(st);
        }
    };
    for (int ch = 0;;) {
        // chunk ch has landed (every wave's part); every wave is done with chunk ch - 1
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        load_chunk(ch + 1, lds1, ch + 1 < nchunks);
        step(lds0, ch);
        if (++ch >= nchunks) break;
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        load_chunk(ch + 1, lds0, ch + 1 < nchunks);
        step(lds1, ch);
        if (++ch >= nchunks) break;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // no load into LDS outlives the workgroup
    write_out<D>(a, t, tot, j);
}

template <int D>
hipError_t launch_attention_d(const AttnArgs& a, bool split, hipStream_t stream) {
    const int64_t R = static_cast<int64_t>(a.G) * a.T;
    const int pairs = a.B * a.KVH;
    if (split) {
        const int tiles = static_cast<int>((R + 15) / 16);
        const dim3 grid(static_cast<unsigned>(a.ns), static_cast<unsigned>(tiles), static_cast<unsigned>(pairs));
        if (a.qkv) attn_split_kernel<D, true><<<grid, dim3(64), 0, stream>>>(a);
        else attn_split_kernel<D, false><<<grid, dim3(64), 0, stream>>>(a);
        if (a.ns > 1)
            attn_combine_kernel<D><<<dim3(static_cast<unsigned>(pairs * R)), dim3(64), 0, stream>>>(a);
    } else {
        const int groups = static_cast<int>((R + 16 * kLoopWaves - 1) / (16 * kLoopWaves));
        attn_loop_kernel<D><<<dim3(static_cast<unsigned>(static_cast<int64_t>(pairs) * groups)),
                              dim3(64 * kLoopWaves), 0, stream>>>(a, groups);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attention(const AttnArgs& a, bool split, hipStream_t stream) {
    if (static_cast<int64_t>(a.B) * a.T == 0) return hipSuccess;
    if (a.D == 128) return launch_attention_d<128>(a, split, stream);
    return launch_attention_d<64>(a, split, stream);
}

}  // namespace w4a8
