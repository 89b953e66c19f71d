// Device helpers shared by the W4A8 kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a8 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (non-temporal hint: read once, do not keep in cache).
__device__ __forceinline__ uint4 load_stream(const uint4* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Raw buffer resources: an SGPR descriptor over [base, base + bytes) plus a
// 32-bit byte offset per lane; reads past `bytes` return zero.  word3 is the
// gfx9 raw-buffer format word.
constexpr int kBufferWord3 = 0x00020000;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufferWord3);
}
// Descriptor over [base + off, base + bytes): a uniform offset moved into the
// SGPR base instead of every lane's offset (saves a VALU add per load); the
// range check then applies to the lane offsets against bytes - off (0 when
// off >= bytes: every read returns zero).  off and bytes are below 2^31; the
// record count is a signed max, which stays a scalar instruction (an unsigned
// saturating subtract would be selected as a VALU op and make the descriptor
// divergent).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_at(const void* base, uint32_t off, uint32_t bytes) {
    const int n = max(static_cast<int>(bytes) - static_cast<int>(off), 0);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(static_cast<const char*>(base)) + off, 0, n,
                                             kBufferWord3);
}
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}
// The same load with the non-temporal cache policy (bit 1 of the buffer
// instruction's cache-policy operand, `nt` on gfx950): for streams read once
// per call (the decode kernels' weights).  Measured on a cold 141.6 MB
// weight pool in the decode kernels' tile order: 73% -> 81% of 8 TB/s.
__device__ __forceinline__ uint4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 2);
    return make_uint4(v.x, v.y, v.z, v.w);
}
// 16 bytes per lane from a buffer straight into LDS (gfx950): lane l's bytes
// land at lds + 16 l (lds wave-uniform).  A plain device function: with the
// builtin written directly in some kernel templates, the host pass drops the
// kernel's launch stub (the library then fails to load).
__device__ __forceinline__ void buf_load16_lds(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, off, 0, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load_u16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(off), 0, 0);
}

// One aligned dword.  Scale rings load the dword holding a lane's 16-bit
// scale and shift it out at the fold: a ring of 16-bit loads makes the
// compiler zero-extend (or copy) each loaded value on the loop latch, which
// waits there for the loads just issued and drains the ring every unrolled
// iteration.
__device__ __forceinline__ uint32_t buf_load_u32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off), 0, 0);
}

// bf16 bits -> fp32 (exact).
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// fp16 bits -> fp32 (exact).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
}

// fp32 -> bf16 bits, round to nearest even; NaN stays NaN (quiet bit set).
// Same rounding as the reference's host conversion (int4_cube_lab/host/bf16.h:17-27)
// and torch's .to(torch.bfloat16): (u + 0x7fff + lsb) >> 16, NaN -> (u >> 16)
// | 0x40.  One v_cvt_pk_bf16_f32, which on MI355X gives exactly that for
// every fp32 input (checked against the integer formula on 2^24 bit
// patterns including ties, subnormals, infinities and NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two fp32 -> two bf16 (low half: a) in one v_cvt_pk_bf16_f32, rounded as
// f32_to_bf16_bits.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float a, float b) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// SwiGLU of one gate/up output pair, rounded the way torch evaluates
// `F.silu(g) * u` on bf16 tensors (the reference's decoder layer,
// npu_ops/python/bench_decode_layer.py:78-81): g and u are first rounded to the
// bf16 GEMM outputs, silu(g) = g / (1 + exp(-g)) is computed in fp32 and rounded
// to bf16, and the product of the two bf16 values is rounded to bf16.
__device__ __forceinline__ uint32_t swiglu_bf16_bits(float g32, float u32) {
    const float g = bf16_bits_to_f32(f32_to_bf16_bits(g32));
    const float u = bf16_bits_to_f32(f32_to_bf16_bits(u32));
    const float s = bf16_bits_to_f32(f32_to_bf16_bits(g / (1.0f + expf(-g))));
    return f32_to_bf16_bits(s * u);
}

// Scale entry -> fp32, for the two scale dtypes the op accepts.
template <bool BF16>
__device__ __forceinline__ float scale_to_f32(uint32_t bits) {
    if constexpr (BF16) return bf16_bits_to_f32(bits);
    else return f16_bits_to_f32(bits);
}

constexpr uint32_t kBf16Tiny = 0x0080u;  // 2^-126, torch.finfo(torch.bfloat16).tiny

// Per-token activation quant helpers (quant_act.hip semantics): the absmax
// of bf16 rows is reduced on the 15 magnitude bits as integers.
__device__ __forceinline__ uint32_t abs_bits_max2(uint32_t u) {
    return max(u & 0x7fffu, (u >> 16) & 0x7fffu);
}

// Scale from the absmax bits; returns bf16 bits of the stored scale.
__device__ __forceinline__ uint32_t scale_from_amax(uint32_t amax_bits) {
    const float amax = bf16_bits_to_f32(amax_bits);
    uint32_t s = f32_to_bf16_bits(amax / 127.0f);
    if ((s & 0x7fffu) == 0u) s = kBf16Tiny;
    return s;
}

__device__ __forceinline__ uint32_t abs_bits_max8(const uint4& v) {
    return max(max(abs_bits_max2(v.x), abs_bits_max2(v.y)), max(abs_bits_max2(v.z), abs_bits_max2(v.w)));
}

// Per-token int8 quant of one element: clamp(rint(x / s), -128, 127) with
// rint = round half to even and the IEEE fp32 quotient.
__device__ __forceinline__ int quant_div(float x, float s) {
    float q = rintf(x / s);
    q = fminf(127.0f, fmaxf(-128.0f, q));
    return static_cast<int>(q);
}

// The row's scale, its reciprocal and half of it.  With s normal (>= 2^-125
// here) and |x| <= 127.25 s (s = bf16(amax / 127) is at least amax / 127
// less one bf16 rounding), y = x * (1/s) lies within 2^-16 of the exact x/s,
// and x/s -- a ratio of two 8-bit significands -- is either a half-integer or
// at least 2^-10 from every half-integer.  So rint(y) is rint(x/s) except at
// exact half-way cases, where the residual x - t*s (exact in an fma) is
// +-s/2 and the even neighbour is taken.  Other scales (subnormal, infinite,
// NaN) divide per element.
struct RowScale {
    float s, r, hs;
    bool fast;
};

__device__ __forceinline__ RowScale row_scale(float s) {
    RowScale q;
    q.s = s;
    q.fast = s >= 0x1p-125f && s <= 3.0e38f;
    q.r = 1.0f / s;
    q.hs = 0.5f * s;
    return q;
}

template <bool FAST>
__device__ __forceinline__ int quant_code(float x, const RowScale& q) {
    if constexpr (!FAST) return quant_div(x, q.s);
    const float t = rintf(x * q.r);
    const float d = fmaf(-t, q.s, x);
    int v = static_cast<int>(t);
    if (fabsf(d) == q.hs && (v & 1)) v += d > 0.0f ? 1 : -1;
    return min(127, max(-128, v));
}

// Two bf16 in one dword -> two int8 codes in the low 16 bits.
template <bool FAST>
__device__ __forceinline__ uint32_t quant2(uint32_t u, const RowScale& q) {
    const int q0 = quant_code<FAST>(__uint_as_float(u << 16), q);
    const int q1 = quant_code<FAST>(__uint_as_float(u & 0xffff0000u), q);
    return (static_cast<uint32_t>(q0) & 0xffu) | ((static_cast<uint32_t>(q1) & 0xffu) << 8);
}

// One packed dword of the repacked weight holds 8 int4 codes: byte j carries
// code k+j in its low nibble and code k+4+j in its high nibble.  Moving each
// nibble into the HIGH half of a byte gives int8 lanes equal to 16*code, with
// no sign handling: lo4 -> codes k..k+3, hi4 -> codes k+4..k+7.  The MFMA then
// accumulates 16*P exactly; the factor is removed in the fp32 epilogue.
__device__ __forceinline__ int unpack_lo4(uint32_t w) { return static_cast<int>((w << 4) & 0xf0f0f0f0u); }
__device__ __forceinline__ int unpack_hi4(uint32_t w) { return static_cast<int>(w & 0xf0f0f0f0u); }

// The reference's mid-group activation planes (one int4 code per nibble,
// even K in the low nibble): q = 16*hi + lo + 8, stored as hi and lo ^ 8.
// Even and odd activation bytes of one dword of each plane: byte j of `ev` is
// (hi nibble 2j << 4) | (lo nibble 2j ^ 8), of `od` the same for nibble 2j+1
// -- the order unpack_lo4 / unpack_hi4 give the weight codes of the same K.
// The lo plane's offset flip (every nibble ^ 8) is one xor for both.
__device__ __forceinline__ void act_pair(uint32_t h, uint32_t l, int& ev, int& od) {
    const uint32_t lx = l ^ 0x88888888u;
    ev = static_cast<int>(((h << 4) & 0xf0f0f0f0u) | (lx & 0x0f0f0f0fu));
    od = static_cast<int>((h & 0xf0f0f0f0u) | ((lx >> 4) & 0x0f0f0f0fu));
}

// 16 packed bytes (32 codes, two 64-K slabs of 16 codes each for one lane) ->
// the two MFMA B operands.
__device__ __forceinline__ void unpack_tile_lane(const uint4 w, v4i& slab0, v4i& slab1) {
    slab0 = v4i{unpack_lo4(w.x), unpack_hi4(w.x), unpack_lo4(w.y), unpack_hi4(w.y)};
    slab1 = v4i{unpack_lo4(w.z), unpack_hi4(w.z), unpack_lo4(w.w), unpack_hi4(w.w)};
}

__device__ __forceinline__ v4i mfma16(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

}  // namespace w4a8
