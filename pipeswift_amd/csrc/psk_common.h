// Helpers shared by the HIP translation units of libpipeswift_kv: error
// reporting for the C ABI, vector load/store widths, element conversions and the
// FP8 E4M3FN quantization used by the append and the attention reader.
#pragma once

#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "pipeswift_kv.h"

namespace psk_detail {

constexpr int kWave = 64;

// ----------------------------------------------------------------------------
// error reporting
// ----------------------------------------------------------------------------

extern thread_local char g_err[512];

inline int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

inline int hip_fail(hipError_t e, const char* what) {
  snprintf(g_err, sizeof(g_err), "%s: %s (hipError_t %d)", what, hipGetErrorString(e), (int)e);
  return (int)e;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? PSK_OK : hip_fail(e, what);
}

// Start of an entry point that launches kernels: clears the thread's message
// and the runtime's last-error slot.  A kernel launch reports its failure only
// through hipGetLastError(), and that slot also keeps the failure of any
// earlier runtime call on this thread (made by another library and already
// returned to its caller); without the reset such an error would be reported
// as a failure of this launch.
inline void begin_device_call() {
  g_err[0] = 0;
  (void)hipGetLastError();
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline int dtype_size(int dt) {
  switch (dt) {
    case PSK_DTYPE_F32: return 4;
    case PSK_DTYPE_F16: return 2;
    case PSK_DTYPE_BF16: return 2;
    case PSK_DTYPE_FP8_E4M3FN: return 1;
    default: return 0;
  }
}

inline int log2_exact(int64_t v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((int64_t(1) << s) < v) ++s;
  return s;
}

// Largest power-of-two byte width <= max_bytes dividing every value in vals.
inline int common_align(const uint64_t* vals, int n, int max_bytes) {
  uint64_t acc = 0;
  for (int i = 0; i < n; ++i) acc |= vals[i];
  int b = max_bytes;
  while (b > 1 && (acc & uint64_t(b - 1))) b >>= 1;
  return b;
}

// ----------------------------------------------------------------------------
// vectors and element conversions
// ----------------------------------------------------------------------------

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

template <int B> struct VecT;
template <> struct VecT<16> { using T = u32x4; };
template <> struct VecT<8> { using T = u32x2; };
template <> struct VecT<4> { using T = uint32_t; };
template <> struct VecT<2> { using T = uint16_t; };
template <> struct VecT<1> { using T = uint8_t; };

template <int B>
__device__ __forceinline__ typename VecT<B>::T vload(const char* p) {
  return *reinterpret_cast<const typename VecT<B>::T*>(p);
}
template <int B>
__device__ __forceinline__ void vstore(char* p, typename VecT<B>::T v) {
  *reinterpret_cast<typename VecT<B>::T*>(p) = v;
}
// Streaming (nontemporal) variants for data touched once per kernel.
template <int B>
__device__ __forceinline__ typename VecT<B>::T vload_nt(const char* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const typename VecT<B>::T*>(p));
}
template <int B>
__device__ __forceinline__ void vstore_nt(char* p, typename VecT<B>::T v) {
  __builtin_nontemporal_store(v, reinterpret_cast<typename VecT<B>::T*>(p));
}

// ---- buffer (V#) loads and stores: an access at or beyond num_records bytes
// of the descriptor returns zeros (loads) or is dropped (stores), so a row
// that must not be touched gets num_records = 0 instead of a branch.
// Dword 3 is the gfx9-family raw-buffer format word; aux 2 = nontemporal.

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t num_records) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(num_records), 0x00020000);
}

template <int B> struct BufIO;
template <> struct BufIO<16> {
  __device__ static u32x4 load(__amdgpu_buffer_rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2); }
  __device__ static void store(u32x4 v, __amdgpu_buffer_rsrc_t r, uint32_t off) { __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 2); }
};
template <> struct BufIO<8> {
  __device__ static u32x2 load(__amdgpu_buffer_rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 2); }
  __device__ static void store(u32x2 v, __amdgpu_buffer_rsrc_t r, uint32_t off) { __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, 2); }
};
template <> struct BufIO<4> {
  __device__ static uint32_t load(__amdgpu_buffer_rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 2); }
  __device__ static void store(uint32_t v, __amdgpu_buffer_rsrc_t r, uint32_t off) { __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, 2); }
};
template <> struct BufIO<2> {
  __device__ static uint16_t load(__amdgpu_buffer_rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 2); }
  __device__ static void store(uint16_t v, __amdgpu_buffer_rsrc_t r, uint32_t off) { __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, 2); }
};
template <> struct BufIO<1> {
  __device__ static uint8_t load(__amdgpu_buffer_rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 2); }
  __device__ static void store(uint8_t v, __amdgpu_buffer_rsrc_t r, uint32_t off) { __builtin_amdgcn_raw_buffer_store_b8(v, r, off, 0, 2); }
};

template <int DT> struct Elt;
template <> struct Elt<PSK_DTYPE_F32> {
  using Bits = uint32_t;
  static constexpr int kSize = 4;
  __device__ static float to_f32(Bits b) { return __uint_as_float(b); }
  __device__ static Bits from_f32(float f) { return __float_as_uint(f); }
};
template <> struct Elt<PSK_DTYPE_BF16> {
  using Bits = uint16_t;
  static constexpr int kSize = 2;
  __device__ static float to_f32(Bits b) { return __uint_as_float(uint32_t(b) << 16); }
  // Round to nearest even; NaN becomes the canonical quiet NaN 0x7FC0.
  __device__ static Bits from_f32(float f) {
    uint32_t u = __float_as_uint(f);
    if (__builtin_isnan(f)) return 0x7FC0;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return Bits(u >> 16);
  }
};
template <> struct Elt<PSK_DTYPE_F16> {
  using Bits = uint16_t;
  static constexpr int kSize = 2;
  __device__ static float to_f32(Bits b) { return float(__builtin_bit_cast(_Float16, b)); }
  __device__ static Bits from_f32(float f) { return __builtin_bit_cast(Bits, _Float16(f)); }
};

// OCP E4M3FN byte for a NaN: 0x7F with the sign bit of the input, which is what
// torch's float -> float8_e4m3fn conversion produces.
__device__ __forceinline__ uint32_t e4m3_nan_byte(float x) {
  return ((__float_as_uint(x) >> 24) & 0x80u) | 0x7Fu;
}

// E4M3FN bytes 0 and 1 (or 2 and 3 with hi) of w -> floats, native conversion.
__device__ __forceinline__ f32x2 e4m3_unpack2(uint32_t w, bool hi) {
  return hi ? __builtin_amdgcn_cvt_pk_f32_fp8(int(w), true) : __builtin_amdgcn_cvt_pk_f32_fp8(int(w), false);
}

// ---- per-tensor scale, prepared once per wave

// The stored byte must be that of the correctly rounded IEEE quotient x / s
// (the reference divides in fp32).  With r = RN(1/s) computed once per wave,
// y = RN(x*r) is within 1.5 ulp of x/s, the residual e = x - y*s is exact in
// one FMA, and z = RN(y + e*r) differs from x/s by at most 1.5 ulp * 2^-24
// before its rounding, which places it on the IEEE quotient unless x/s lies
// within that distance of a rounding midpoint (Markstein's correction step).
// The host restatement in oracle/quant_check.c sweeps every bf16 and f16 input
// against the scale RN(a/448) of every finite bf16 / f16 amax a (4.2e9 cases)
// plus 2e8 sampled fp32 pairs: z equals the IEEE quotient bit for bit whenever
// |x/s| >= 2^-20 and gives the same E4M3 byte in every case.  Where the gate
// below holds, the only inexact quotients are:
//   * |x| < 2^-100: the quotient is below 2^-20 and converts to a signed zero,
//     so only its sign matters, which copysign(., y) keeps (also for x = +-0);
//   * y = +-inf or NaN (x infinite, NaN, or the quotient overflows): y itself
//     is the right input to the clamp.
// Any other scale (|s| outside [2^-80, 2^100): 0, inf, NaN, tiny) takes the
// plain IEEE division.  At s == 1.0 (the reference's fixed scale) r = 1, y = x
// and e = 0, so the quotient is x.
// QScale keeps |s| and 1 / |s|; the sign of a negative scale (which no caller
// passes, but the C ABI accepts) is a byte mask that QuantConv puts onto the
// signs of its outputs, so the quotients it divides are never negative.
struct QScale {
  float s;        // |scale|
  float r;        // RN(1 / |scale|)
  bool fast;
  uint32_t neg;   // 0x80808080 for a negative scale, else 0
};

__device__ __forceinline__ QScale make_qscale(float s) {
  QScale q;
  q.s = __builtin_fabsf(s);
  q.r = 1.0f / q.s;
  q.fast = q.s >= 0x1p-80f && q.s < 0x1p100f;
  q.neg = __builtin_signbit(s) ? 0x80808080u : 0u;
  return q;
}

// For a scale that is the same in every lane of the wave.  The range test then
// becomes a scalar branch: without it the compiler cannot tell that the test is
// uniform, and evaluates both the fast path and the IEEE divisions for every
// element, selecting per lane.
__device__ __forceinline__ QScale make_qscale_uniform(float s) {
  QScale q = make_qscale(s);
  q.fast = __builtin_amdgcn_readfirstlane(int(q.fast)) != 0;
  return q;
}

// Exact for s == 1.0 as well: r = 1, y = x, e = 0.  BOUNDED: the caller
// knows that y is finite or NaN (x is never infinite on this path and |x / s|
// cannot overflow, as for a tile divided by its own amax / 448), so the
// select that passes an infinite y through is left out.
template <bool BOUNDED = false>
__device__ __forceinline__ float div_fast(float x, const QScale& q) {
  const float y = x * q.r;
  const float e = __builtin_fmaf(-y, q.s, x);
  const float z = __builtin_copysignf(__builtin_fmaf(e, q.r, y), y);
  if constexpr (BOUNDED) return z;  // a NaN y gives a NaN z with y's sign
  return __builtin_fabsf(y) < __builtin_inff() ? z : y;
}

// ---- conversion policies: In vector (IN_B bytes) -> Out vector (OUT_B bytes)

template <int B>
struct CopyConv {
  static constexpr int IN_B = B;
  static constexpr int OUT_B = B;
  using In = typename VecT<B>::T;
  using Out = typename VecT<B>::T;
  __device__ static Out apply(In v, const QScale&) { return v; }
  __device__ static Out zero() { return Out(0); }
};

// What a NaN quotient stores.  kNanClampMin: the byte of -448 (0xFE), which
// is what the reference's append stores: its clamp min(max(x, -448), 448) is
// Triton's tl.minimum / tl.maximum, whose default PropagateNan.NONE lowers to
// minnum / maxnum, and maxnum(NaN, -448) = -448 (reshape_and_cache.py:70-75;
// triton/language/core.py:2506,2528, semantic.py:380-381 in Triton 3.6).
// kNanTorch: 0x7F with the input's sign, torch's clamp-then-convert, which the
// reference's query quantizer uses (fp8_kv.py:75-77).
enum NanPolicy { kNanClampMin = 0, kNanTorch = 1 };

// E input elements of type IN_DT -> E E4M3FN bytes, q = e4m3(clamp(x / scale)),
// in sign-magnitude form (E4M3 is sign-magnitude and scales are positive):
//   m = |x| / s    (div_fast's sequence on |x|; |x| is a free source
//                   modifier, and a non-negative quotient needs no copysign)
//   byte = e4m3(min(m, 448)) | sign(x)
// One v_min_f32 both clamps and handles the infinite quotients: IEEE-mode min
// returns the non-NaN operand, so the NaN that the correction step makes of an
// infinite quotient (|x| infinite, or |x| / s overflowing) becomes 448, as the
// clamp of an infinite quotient does.  A NaN quotient (a NaN input, or 0/0,
// inf/inf and x/NaN for a scale outside the gate) is rewritten by the policy
// afterwards (rare path).  Every element costs the multiply and two FMAs of
// the division, one min, half a packed convert and the sign's move onto the
// byte.  Scales outside [2^-80, 2^100) take the IEEE division of |x| by |s|.
template <int IN_DT, int E, int NAN_POLICY = kNanClampMin>
struct QuantConv {
  using EltT = Elt<IN_DT>;
  static constexpr int IN_B = E * EltT::kSize;
  static constexpr int OUT_B = E;
  using In = typename VecT<IN_B>::T;
  using Out = typename VecT<OUT_B>::T;
  __device__ static Out apply(In v, const QScale& qs) {
    typename EltT::Bits e[E];
    __builtin_memcpy(e, &v, sizeof(v));
    float m[E];
    bool any_nan = false;
    if (__builtin_expect(qs.fast, 1)) {
      // NaN inputs: with r finite and positive, y = |x| r is NaN exactly
      // when x is (an infinite x gives an infinite y), and y's bits read as
      // unsigned exceed the infinity's only for a NaN -- one integer maximum
      // over the y (three-input v_max3_u32), then one compare
      uint32_t ymax = 0;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const float x = EltT::to_f32(e[i]);
        const float a = __builtin_fabsf(x);
        const float y = a * qs.r;
        ymax = __builtin_elementwise_max(ymax, __float_as_uint(y));
        const float r = __builtin_fmaf(-y, qs.s, a);
        m[i] = __builtin_fmaf(r, qs.r, y);
      }
      any_nan = ymax > 0x7F800000u;
    } else {
      // scales outside [2^-80, 2^100) (0, inf, NaN, subnormal): IEEE division.
      // The empty volatile asm keeps this a branch: otherwise the compiler
      // computes both paths for every element and selects.
      asm volatile("");
#pragma unroll
      for (int i = 0; i < E; ++i) {
        m[i] = __builtin_fabsf(EltT::to_f32(e[i])) / qs.s;
        any_nan |= __builtin_isnan(m[i]);
      }
    }
    // Clamp: m is +0..+inf or a NaN, and for such bit patterns the unsigned
    // order is the float order with every NaN above +inf, so one v_min_u32
    // against 448's bits clamps and sends inf and NaN to 448 (a float min
    // would first canonicalize its input, one more instruction).
    uint32_t c[E];
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const uint32_t b = __float_as_uint(m[i]);
      c[i] = b < 0x43E00000u ? b : 0x43E00000u;
    }
    // Four elements per word: two packed converts into its halves, then the
    // inputs' sign bits onto the four bytes.
    constexpr int NW = (E + 3) / 4;
    uint32_t q[NW];
#pragma unroll
    for (int g = 0; g < NW; ++g) {
      const int i = 4 * g;
      // the high half of `old` is overwritten below or not stored
      uint32_t w = uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(c[i]),
                                                             i + 1 < E ? __uint_as_float(c[i + 1]) : 0.0f,
                                                             int(c[i]), false));
      if (i + 2 < E)
        w = uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(c[i + 2]),
                                                      i + 3 < E ? __uint_as_float(c[i + 3]) : 0.0f, int(w), true));
      q[g] = w;
    }
    if constexpr (EltT::kSize == 2 && E >= 2) {
      // the high byte of every 16-bit input holds its sign bit
      uint32_t in[E / 2];
      __builtin_memcpy(in, &v, sizeof(in));
#pragma unroll
      for (int g = 0; g < NW; ++g) {
        const uint32_t sg = E >= 4 ? __builtin_amdgcn_perm(in[2 * g + 1], in[2 * g], 0x07050301u)
                                   : __builtin_amdgcn_perm(0u, in[0], 0x0C0C0301u);
        q[g] |= (sg ^ qs.neg) & 0x80808080u;
      }
    } else {
#pragma unroll
      for (int i = 0; i < E; ++i)
        q[i / 4] |= (((uint32_t(e[i]) >> (8 * EltT::kSize - 8)) ^ qs.neg) & 0x80u) << (8 * (i % 4));
    }
    if (__builtin_expect(any_nan, 0)) {
      // the NaN quotients: NaN inputs on the fast path (its NaN m of an
      // infinite quotient is not one), NaN m on the IEEE path
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const float x = EltT::to_f32(e[i]);
        if (qs.fast ? __builtin_isnan(x) : __builtin_isnan(m[i])) {
          const uint32_t nb = NAN_POLICY == kNanClampMin ? 0xFEu : e4m3_nan_byte(x);
          const int sh = 8 * (i % 4);
          q[i / 4] = (q[i / 4] & ~(0xFFu << sh)) | (nb << sh);
        }
      }
    }
    Out r;
    __builtin_memcpy(&r, q, sizeof(r));
    return r;
  }
  __device__ static Out zero() { return Out(0); }
};

// E E4M3FN bytes -> E elements of OUT_DT, y = round(float(q) * scale).
template <int OUT_DT, int E>
struct DequantConv {
  using EltT = Elt<OUT_DT>;
  static constexpr int IN_B = E;
  static constexpr int OUT_B = E * EltT::kSize;
  using In = typename VecT<IN_B>::T;
  using Out = typename VecT<OUT_B>::T;
  __device__ static Out apply(In v, const QScale& qs) {
    uint8_t q[E];
    __builtin_memcpy(q, &v, sizeof(v));
    typename EltT::Bits o[E];
    if constexpr (E == 1) {
      o[0] = EltT::from_f32(e4m3_unpack2(uint32_t(q[0]), false).x * qs.s);
    } else {
#pragma unroll
      for (int i = 0; i < E; i += 2) {
        const f32x2 f = e4m3_unpack2(uint32_t(q[i]) | (uint32_t(q[i + 1]) << 8), false);
        o[i] = EltT::from_f32(f.x * qs.s);
        o[i + 1] = EltT::from_f32(f.y * qs.s);
      }
    }
    Out r;
    __builtin_memcpy(&r, o, sizeof(r));
    return r;
  }
  __device__ static Out zero() { return Out(0); }
};

}  // namespace psk_detail
