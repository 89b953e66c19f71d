// The staged-activation variants of the decode GEMM (decode_kernel.h, SA > 0):
// built in their own translation unit so that they compile in parallel with
// gemm_decode.hip.
#include "decode_kernel.h"

namespace w4a8 {
namespace dec {

template <int MODE>
hipError_t dispatch_staged(const DecodeParams& p, const DecodeConfig& c, bool sbf16, hipStream_t s) {
    if (c.D != 4 || p.M < 1 || p.M > 8) return hipErrorInvalidValue;
    // 16-byte lane loads per pass: M rows of 512 bytes over 64 lanes
    const int sa = p.M <= 2 ? 1 : (p.M <= 4 ? 2 : 4);
    if (c.CPW == 2) {
        if (sa == 1) return launch_v<1, 2, 4, MODE, 1>(p, c.KW, sbf16, s);
        if (sa == 2) return launch_v<1, 2, 4, MODE, 2>(p, c.KW, sbf16, s);
        return launch_v<1, 2, 4, MODE, 4>(p, c.KW, sbf16, s);
    }
    if constexpr (MODE != 2) {
        if (c.CPW == 1) {
            if (sa == 1) return launch_v<1, 1, 4, MODE, 1>(p, c.KW, sbf16, s);
            if (sa == 2) return launch_v<1, 1, 4, MODE, 2>(p, c.KW, sbf16, s);
            return launch_v<1, 1, 4, MODE, 4>(p, c.KW, sbf16, s);
        }
    }
    return hipErrorInvalidValue;
}

template hipError_t dispatch_staged<0>(const DecodeParams&, const DecodeConfig&, bool, hipStream_t);
template hipError_t dispatch_staged<1>(const DecodeParams&, const DecodeConfig&, bool, hipStream_t);
template hipError_t dispatch_staged<2>(const DecodeParams&, const DecodeConfig&, bool, hipStream_t);

}  // namespace dec
}  // namespace w4a8
