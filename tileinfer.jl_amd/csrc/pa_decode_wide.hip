// The 48- and 64-row decode / verify variants (G x n packed query rows > 32), built in a
// translation unit of their own without VGPR-form MFMA: their accumulators (up to 128
// registers) live in AGPRs, which leaves the 256 architectural VGPRs for the query
// operands and the software pipeline. The softmax rescale that touches the accumulators
// is lazy (rare), so AGPR copies stay off the steady-state path.
#include "pa_decode.hpp"

using namespace ti;
using namespace ti_decode;

namespace {

template <int D, bool INT8, bool PG16>
void launch_wide(const DecodeParams &p, int rowb, dim3 grid, hipStream_t s) {
    if (rowb == 3) decode_kernel<D, 3, INT8, PG16, 4><<<grid, 256, 0, s>>>(p);
    else decode_kernel<D, 4, INT8, PG16, 4><<<grid, 256, 0, s>>>(p);
}

}  // namespace

void ti_launch_decode_wide(const DecodeParams &p, int D, int rowb, bool int8, bool pg16, dim3 grid,
                           hipStream_t s) {
    if (D == 128) {
        if (int8) { if (pg16) launch_wide<128, true, true>(p, rowb, grid, s); else launch_wide<128, true, false>(p, rowb, grid, s); }
        else { if (pg16) launch_wide<128, false, true>(p, rowb, grid, s); else launch_wide<128, false, false>(p, rowb, grid, s); }
    } else {
        if (int8) { if (pg16) launch_wide<64, true, true>(p, rowb, grid, s); else launch_wide<64, true, false>(p, rowb, grid, s); }
        else { if (pg16) launch_wide<64, false, true>(p, rowb, grid, s); else launch_wide<64, false, false>(p, rowb, grid, s); }
    }
}
