// Shared device helpers for the MoC HIP kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moc {

enum DType : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };
// What `alpha` holds: weights (ROUTE_ALPHA); logits whose softmax / exp the
// kernels form (ROUTE_SOFTMAX / ROUTE_EXP); or weights that already are the
// softmax / exp of the logits (ROUTE_SOFTMAX_W / ROUTE_EXP_W), used as they are
// in the forward, with the backward's dalpha the logits gradient.
enum Route : int {
  ROUTE_ALPHA = 0,
  ROUTE_SOFTMAX = 1,
  ROUTE_EXP = 2,
  ROUTE_SOFTMAX_W = 3,
  ROUTE_EXP_W = 4
};
// activation the kernels apply to alpha before the mixture
__host__ __device__ inline int route_form(int r) { return r >= ROUTE_SOFTMAX_W ? ROUTE_ALPHA : r; }
// activation whose gradient the backward applies to dalpha
__host__ __device__ inline int route_grad(int r) { return r >= ROUTE_SOFTMAX_W ? r - 2 : r; }

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// fp32 -> bf16 bits, round to nearest even (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
  __bf16 h = static_cast<__bf16>(v);
  return __builtin_bit_cast(uint16_t, h);
}

// Round v to the precision of storage dtype dt and return it as fp32.
__device__ __forceinline__ float round_to(float v, int dt) {
  if (dt == DT_BF16) return bf16_to_f32(f32_to_bf16(v));
  if (dt == DT_F16) return static_cast<float>(static_cast<_Float16>(v));
  return v;
}

__device__ __forceinline__ float load_any(const void* p, int dt, int64_t i) {
  if (dt == DT_F32) return static_cast<const float*>(p)[i];
  if (dt == DT_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  return static_cast<float>(static_cast<const _Float16*>(p)[i]);
}

__device__ __forceinline__ void store_any(void* p, int dt, int64_t i, float v) {
  if (dt == DT_F32) {
    static_cast<float*>(p)[i] = v;
  } else if (dt == DT_BF16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
  } else {
    static_cast<_Float16*>(p)[i] = static_cast<_Float16>(v);
  }
}

// Logistic function with the hardware exp2 / reciprocal (v_exp_f32, v_rcp_f32).
__device__ __forceinline__ float sigmoid_f(float p) {
  const float e = __builtin_amdgcn_exp2f(-p * 1.4426950408889634f);
  return __builtin_amdgcn_rcpf(1.0f + e);
}

// Sequence layout of the flat token axis [0, n_tokens).
//   fixed : sequences of seq_len tokens back to back ([B,T,D] viewed as [B*T,D])
//   packed: token n of sequence j lies in [cu[j], cu[j+1]).
// The packed axis is cut into the segments [0, cu[0]), [cu[0], cu[1]), ...,
// [cu[n], n_tokens); tokens outside every sequence therefore form segments of
// their own.  bounds() returns [lo, hi) of the segment holding token t,
// clamped to [0, n_tokens] and always containing t, so every access derived
// from it stays inside the token axis whatever cu_seqlens holds.
struct SeqLayout {
  const void* cu;
  int cu64;
  int64_t n_seqs;
  int64_t seq_len;
  int64_t n_tokens;

  // cu_seqlens is read-only for a kernel's lifetime: read it through the
  // constant address space so that wave-uniform reads become scalar loads.
  typedef const __attribute__((address_space(4))) int32_t c_i32;
  typedef const __attribute__((address_space(4))) int64_t c_i64;
  __device__ __forceinline__ int64_t cu_at(int64_t j) const {
    return cu64 ? ((c_i64*)cu)[j] : static_cast<int64_t>(((c_i32*)cu)[j]);
  }

  __device__ __forceinline__ void bounds(int64_t t, int64_t& lo, int64_t& hi) const {
    if (cu == nullptr) {
      if (((t | seq_len) >> 32) == 0) {  // 32-bit division where it suffices
        const uint32_t q = static_cast<uint32_t>(t) / static_cast<uint32_t>(seq_len);
        lo = static_cast<int64_t>(q) * seq_len;
      } else {
        lo = (t / seq_len) * seq_len;
      }
      hi = lo + seq_len;
      if (hi > n_tokens) hi = n_tokens;
      return;
    }
    const int64_t c0 = cu_at(0);
    if (t < c0) {
      lo = 0;
      hi = c0;
    } else {
      // largest a in [0, n_seqs] with cu[a] <= t
      int64_t a = 0, b = n_seqs;
      while (a < b) {
        const int64_t m = (a + b + 1) >> 1;
        if (cu_at(m) <= t) a = m; else b = m - 1;
      }
      lo = cu_at(a);
      hi = (a < n_seqs) ? cu_at(a + 1) : n_tokens;
    }
    if (lo < 0) lo = 0;
    if (lo > t) lo = t;
    if (hi > n_tokens) hi = n_tokens;
    if (hi <= t) hi = t + 1;
  }

  // Smallest segment start >= lo (segment starts: 0, the cu entries, in order),
  // or n_tokens if there is none below n_tokens.  Called with wave-uniform
  // arguments, so its loads are scalar.
  __device__ __forceinline__ int64_t next_start(int64_t lo) const {
    if (lo <= 0) return 0;
    if (lo >= n_tokens) return n_tokens;
    if (cu == nullptr) {
      const int64_t k = (lo + seq_len - 1) / seq_len;
      const int64_t b = k * seq_len;
      return b < n_tokens ? b : n_tokens;
    }
    // first j in [0, n_seqs] with cu[j] >= lo
    int64_t a = 0, e = n_seqs + 1;
    while (a < e) {
      const int64_t m = (a + e) >> 1;
      if (cu_at(m) < lo) a = m + 1; else e = m;
    }
    if (a > n_seqs) return n_tokens;
    const int64_t b = cu_at(a);
    return (b < n_tokens && b >= lo) ? b : n_tokens;
  }
};

}  // namespace moc
