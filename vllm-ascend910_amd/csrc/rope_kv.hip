// Rotary embedding of q and k fused with the KV-cache append (gfx950).
//
// One launch for what the decoder layer otherwise runs as a dozen elementwise
// kernels per projection output (float casts, four products, a difference, a
// sum, a concatenation, a bf16 cast for q and again for k, then an indexed
// copy into each cache).  For token t of sequence b at position p = pos[0] + t
// and pair index i < D/2 of head h (rotate-half form, x1 = x[i], x2 = x[i+D/2],
// c = cos[p, i], s = sin[p, i] in fp32):
//   y[i]       = bf16( fl(x1 * c) - fl(x2 * s) )
//   y[i + D/2] = bf16( fl(x2 * c) + fl(x1 * s) )
// each product and the sum rounded to fp32 separately (no fused multiply-add),
// then round-to-nearest-even -- the sequence torch evaluates for
// `cat([x1*c - x2*s, x2*c + x1*s]).to(bfloat16)` on float tensors.  An
// optional projection bias is added first, x = bf16(x + bias), as torch adds
// two bf16 tensors (q, k and v alike).  The q heads
// go to q_out [B, T, H, D]; the k heads to k_cache[b, h, :, p] and the raw v
// heads to v_cache[b, h, p, :] through per-dimension strides, so either cache
// layout ([B, KVH, D, L] or [B, KVH, L, D]) is served.  The position is read
// on the device, so a captured decode step advances with it; a token whose
// position falls outside [0, L) writes nothing to the caches and zeros to q.
#include "common.h"
#include "launch.h"

namespace w4a8 {
namespace {

// Workgroup (token, head): heads 0 .. H-1 are q, H .. H+KVH-1 are k (both
// rotated, one pair per thread), the rest v (two elements per thread).
__global__ __launch_bounds__(64) void rope_kv_kernel(const RopeKvArgs a) {
#pragma clang fp contract(off)
    const int tok = static_cast<int>(blockIdx.x);      // b * T + t
    const int hh = static_cast<int>(blockIdx.y);
    const int b = tok / a.T;
    const int t = tok - b * a.T;
    const int64_t p = a.pos[0] + t;
    const int half = a.D / 2;
    const bool inside = p >= 0 && p < a.L;
    const uint16_t* x = a.qkv + static_cast<int64_t>(tok) * a.ldq + hh * a.D;
    const uint16_t* bias = a.bias ? a.bias + hh * a.D : nullptr;
    // x (+ bias, rounded to bf16 as a bf16 add rounds it)
    auto in = [&](int d) {
        const float v = bf16_bits_to_f32(x[d]);
        return bias ? bf16_bits_to_f32(f32_to_bf16_bits(v + bf16_bits_to_f32(bias[d]))) : v;
    };
    if (hh >= a.H + a.KVH) {
        if (!inside) return;
        uint16_t* vr = a.v_cache + b * a.vs[0] + (hh - a.H - a.KVH) * a.vs[1] + p * a.vs[2];
        for (int d = threadIdx.x; d < a.D; d += blockDim.x)
            vr[d * a.vs[3]] = static_cast<uint16_t>(f32_to_bf16_bits(in(d)));
        return;
    }
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        uint16_t o1 = 0, o2 = 0;   // no angle row and no cache slot: q reads as zero
        if (inside) {
            const float x1 = in(i), x2 = in(i + half);
            const float c = a.cos[p * a.ldc + i], s = a.sin[p * a.ldc + i];
            const float y1 = x1 * c - x2 * s;
            const float y2 = x2 * c + x1 * s;
            o1 = static_cast<uint16_t>(f32_to_bf16_bits(y1));
            o2 = static_cast<uint16_t>(f32_to_bf16_bits(y2));
        }
        if (hh < a.H) {
            uint16_t* q = a.q_out + (static_cast<int64_t>(tok) * a.H + hh) * a.D;
            q[i] = o1;
            q[i + half] = o2;
        } else if (inside) {
            uint16_t* k = a.k_cache + b * a.ks[0] + (hh - a.H) * a.ks[1] + p * a.ks[3];
            k[i * a.ks[2]] = o1;
            k[(i + half) * a.ks[2]] = o2;
        }
    }
}

}  // namespace

hipError_t launch_rope_kv(const RopeKvArgs& a, hipStream_t stream) {
    const int64_t tokens = static_cast<int64_t>(a.B) * a.T;
    if (tokens <= 0) return hipSuccess;
    rope_kv_kernel<<<dim3(static_cast<unsigned>(tokens), static_cast<unsigned>(a.H + 2 * a.KVH)), dim3(64), 0,
                     stream>>>(a);
    return hipGetLastError();
}

}  // namespace w4a8
