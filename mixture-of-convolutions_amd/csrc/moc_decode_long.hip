// Decode step on the matrix cores for 9 to 16 taps: the kernels of moc_decode.h
// instantiated in a translation unit of their own (built in parallel with the
// 2-8 tap ones).
#include "moc_decode.h"

namespace moc {
namespace decode {

template <bool FUSED>
bool launch_long(const void* x, const void* alpha, int routing, const void* basis, void* cache,
                 void* y, int64_t B, int64_t D, int64_t K, int64_t S, int act, const void* z,
                 const void* router, int64_t Z, hipStream_t st) {
  switch (S) {
#define MOC_DEC_LONG(S_) \
    case S_: return launch_s<S_, FUSED>(x, alpha, routing, basis, cache, y, B, D, K, act, z, router, Z, st);
    MOC_DEC_LONG(9)
    MOC_DEC_LONG(10)
    MOC_DEC_LONG(11)
    MOC_DEC_LONG(12)
    MOC_DEC_LONG(13)
    MOC_DEC_LONG(14)
    MOC_DEC_LONG(15)
    MOC_DEC_LONG(16)
#undef MOC_DEC_LONG
    default: return false;
  }
}

template bool launch_long<false>(const void*, const void*, int, const void*, void*, void*, int64_t,
                                 int64_t, int64_t, int64_t, int, const void*, const void*, int64_t,
                                 hipStream_t);
template bool launch_long<true>(const void*, const void*, int, const void*, void*, void*, int64_t,
                                int64_t, int64_t, int64_t, int, const void*, const void*, int64_t,
                                hipStream_t);

}  // namespace decode
}  // namespace moc
