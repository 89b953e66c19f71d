// extern "C" wrappers over the reference's own C++ CPU reference
// (int4_cube_lab/host/gemm_ref.cpp, bf16.h, npu_ops/kernel/mg_kgeom.h), so the
// Python tests can call it.  TEST INFRASTRUCTURE ONLY: built by oracle/Makefile
// from the reference sources where they lie, into oracle/_ref/.  Nothing is
// copied from the reference; this file only adapts pointer arguments to the
// std::vector signatures of gemm_ref.h.
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <vector>

#include <omp.h>

#include "bf16.h"
#include "gemm_ref.h"
#include "mg_kgeom.h"

extern "C" {

// OpenMP team size of the reference's parallel loops (for timing: the thread
// count a baseline states is the one it ran with).
void ref_set_threads(int n) { omp_set_num_threads(n); }
int ref_max_threads(void) { return omp_get_max_threads(); }

void ref_fp32_to_bf16(const float* x, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = FP32ToBF16(x[i]);
}

uint32_t ref_num_groups(uint32_t K, uint32_t gk) { return mgk::NumGroups(K, gk); }
uint32_t ref_group_real(uint32_t g, uint32_t K, uint32_t gk) { return mgk::GroupRealElems(g, K, gk); }
uint32_t ref_group_offset(uint32_t g, uint32_t gk) { return mgk::GroupOffsetElems(g, gk, mgk::kCubeKElemsInt4); }
uint32_t ref_kpad(uint32_t K, uint32_t gk) { return mgk::KPadElems(K, gk, mgk::kCubeKElemsInt4); }

void ref_pack_int4(const int8_t* v, size_t rows, size_t cols, int8_t* out) {
    std::vector<int8_t> in(v, v + rows * cols);
    std::vector<int8_t> p = PackInt4(in, rows, cols);
    std::memcpy(out, p.data(), p.size());
}

void ref_pack_int4_grouped(const int8_t* v, size_t rows, uint32_t K, uint32_t gk, int8_t* out) {
    std::vector<int8_t> in(v, v + rows * K);
    std::vector<int8_t> p = PackInt4Grouped(in, rows, K, gk);
    std::memcpy(out, p.data(), p.size());
}

void ref_weight_ksum_per_group(const int8_t* w, size_t rows, size_t cols, size_t gk, int32_t* out) {
    std::vector<int8_t> in(w, w + rows * cols);
    std::vector<int32_t> k = WeightKSumPerGroup(in, rows, cols, gk);
    std::memcpy(out, k.data(), k.size() * sizeof(int32_t));
}

void ref_act_ksum_neg_per_group(const int8_t* a, size_t rows, size_t cols, size_t gk, int32_t* out) {
    std::vector<int8_t> in(a, a + rows * cols);
    std::vector<int32_t> k = ActKSumNegPerGroup(in, rows, cols, gk);
    std::memcpy(out, k.data(), k.size() * sizeof(int32_t));
}

void ref_split_planes_grouped(const int8_t* a, size_t rows, uint32_t K, uint32_t gk, int8_t* hi, int8_t* lo) {
    std::vector<int8_t> in(a, a + rows * K), h, l;
    SplitInt8ToInt4PlanesGrouped(in, rows, K, gk, h, l);
    std::memcpy(hi, h.data(), h.size());
    std::memcpy(lo, l.data(), l.size());
}

// y[m,n] = bf16( sum_g float(sum_{k in g} a*(w - wz)) * ws[g,n] * as[g,m] ).
// a_scale_g [G, mp], w_scale_g / w_zero_g [G, N] bf16 bits; w_zero_g may be NULL.
void ref_midgroup_gemm(const int8_t* a_q, const uint16_t* a_scale_g, const int8_t* w_q,
                       const uint16_t* w_scale_g, const uint16_t* w_zero_g, uint16_t* y,
                       uint32_t M, uint32_t N, uint32_t K, uint32_t gk, uint32_t mp) {
    const size_t G = mgk::NumGroups(K, gk);
    const uint32_t Mp = mp ? mp : M;
    std::vector<int8_t> a(a_q, a_q + size_t(M) * K), w(w_q, w_q + size_t(N) * K);
    std::vector<uint16_t> as(a_scale_g, a_scale_g + G * Mp), ws(w_scale_g, w_scale_g + G * N), wz, out;
    if (w_zero_g) wz.assign(w_zero_g, w_zero_g + G * N);
    ReferenceMidGroupGemm(a, as, w, ws, wz, out, M, N, K, gk, Mp);
    std::memcpy(y, out.data(), out.size() * sizeof(uint16_t));
}

void ref_perchannel_gemm(const int8_t* a_q, const uint16_t* a_scale, const int8_t* w_q,
                         const uint16_t* w_scale, uint16_t* y, uint32_t M, uint32_t N, uint32_t K) {
    std::vector<int8_t> a(a_q, a_q + size_t(M) * K), w(w_q, w_q + size_t(N) * K);
    std::vector<uint16_t> as(a_scale, a_scale + M), ws(w_scale, w_scale + N), out;
    ReferencePerchannelGemm(a, as, w, ws, out, M, N, K);
    std::memcpy(y, out.data(), out.size() * sizeof(uint16_t));
}

}  // extern "C"
