// MFMA forward / backward kernels instantiated for kernel size S = 13 (single
// launches; the grouped and prefill entries take 2 to 8 taps).
#include "moc_mfma_launch.h"

namespace moc {
namespace mfma {

template void launch_fwd<13>(const Problem&, const void*, const void*, const void*, void*,
                              hipStream_t);
template void launch_bwd<13>(const Problem&, const void*, const void*, const void*, const void*,
                              void*, float*, float*, float*, hipStream_t);
template void launch_dx_pass<13>(const Problem&, const void*, const void*, const uint16_t*,
                                  const uint16_t*, void*, float*, hipStream_t);
template void launch_taps_chunk<13>(const Problem&, const void*, const void*, const uint16_t*,
                                     const uint16_t*, float*, float*, float*, hipStream_t);

}  // namespace mfma
}  // namespace moc
