// Decode step on the matrix cores: the shape dispatch and the library-facing
// entries (the kernel and its launch templates are in moc_decode.h).
#include "moc_decode.h"

namespace moc {
namespace decode {

// Returns false (nothing launched) for a shape the kernels are not built for;
// decode_supported / decode_step_supported admit none of them.
template <bool FUSED>
bool launch_any(const void* x, const void* alpha, int routing, const void* basis, void* cache,
                void* y, int64_t B, int64_t D, int64_t K, int64_t S, int act, const void* z,
                const void* router, int64_t Z, hipStream_t st) {
  switch (S) {
    case 2: return launch_s<2, FUSED>(x, alpha, routing, basis, cache, y, B, D, K, act, z, router, Z, st);
    case 3: return launch_s<3, FUSED>(x, alpha, routing, basis, cache, y, B, D, K, act, z, router, Z, st);
    case 4: return launch_s<4, FUSED>(x, alpha, routing, basis, cache, y, B, D, K, act, z, router, Z, st);
    case 5: return launch_s<5, FUSED>(x, alpha, routing, basis, cache, y, B, D, K, act, z, router, Z, st);
    case 6: return launch_s<6, FUSED>(x, alpha, routing, basis, cache, y, B, D, K, act, z, router, Z, st);
    case 7: return launch_s<7, FUSED>(x, alpha, routing, basis, cache, y, B, D, K, act, z, router, Z, st);
    case 8: return launch_s<8, FUSED>(x, alpha, routing, basis, cache, y, B, D, K, act, z, router, Z, st);
    default:
      return S <= 16 && launch_long<FUSED>(x, alpha, routing, basis, cache, y, B, D, K, S, act, z, router,
                                           Z, st);
  }
}

}  // namespace decode

bool decode_supported(int64_t B, int64_t D, int64_t K, int64_t S, int x_dt, int a_dt, int b_dt,
                      int64_t cs_b, int64_t cs_d, int64_t cs_s) {
  const bool s_ok = S >= 2 && S <= 16;
  // buffers are addressed with 32-bit byte offsets
  const int64_t lim = int64_t(1) << 31;
  return x_dt == DT_BF16 && a_dt == DT_BF16 && b_dt == DT_BF16 && s_ok && K <= 64 && K % 4 == 0 &&
         D % 2 == 0 && cs_s == 1 && cs_d == S && cs_b == D * S && 16 * D * S * 2 < lim &&
         B * K * 2 < lim && K * S * D * 2 < lim;
}

bool launch_decode(const void* x, const void* alpha, int routing, const void* basis, void* cache,
                   void* y, int64_t B, int64_t D, int64_t K, int64_t S, int activation,
                   hipStream_t st) {
  return decode::launch_any<false>(x, alpha, routing, basis, cache, y, B, D, K, S, activation, nullptr,
                            nullptr, 0, st);
}

bool decode_step_supported(int64_t B, int64_t D, int64_t Z, int64_t K, int64_t S) {
  const int64_t lim = int64_t(1) << 31;
  return decode_supported(B, D, K, S, DT_BF16, DT_BF16, DT_BF16, D * S, S, 1) && K <= 32 && Z >= 64 &&
         Z % 64 == 0 && 16 * Z * 2 < lim && K * Z * 2 < lim;
}

bool launch_decode_step(const void* z, const void* router, const void* x, const void* basis,
                        void* cache, void* y, int64_t B, int64_t Z, int64_t D, int64_t K,
                        int64_t S, int activation, int routing, hipStream_t st) {
  return decode::launch_any<true>(x, nullptr, routing, basis, cache, y, B, D, K, S, activation, z, router,
                           Z, st);
}

}  // namespace moc
