// MFMA forward / backward kernels instantiated for kernel size S = 5.
#include "moc_mfma_launch.h"

namespace moc {
namespace mfma {

template void launch_fwd<5>(const Problem&, const void*, const void*, const void*, void*,
                             hipStream_t);
template void launch_bwd<5>(const Problem&, const void*, const void*, const void*, const void*,
                             void*, float*, float*, float*, hipStream_t);
template void launch_fwd_layers<5>(const Problem&, const LayerOps*, int, hipStream_t);
template void launch_bwd_layers<5>(const Problem&, const LayerOps*, int, hipStream_t);
template void launch_fwd_pre<5>(const Problem&, const void*, const void*, const void*, void*,
                                 const Pre&, hipStream_t);
template void launch_bwd_pre<5>(const Problem&, const void*, const void*, const void*, const void*,
                                 void*, float*, float*, const Pre&, hipStream_t);

}  // namespace mfma
}  // namespace moc
