// Shared device helpers for the gfx950 attention kernels.
//
// Numeric contract for RoPE: the rotation is evaluated exactly as PyTorch eager
// evaluates kempnerforge/model/position.py:65-71 — the float32 tables are cast to
// the input dtype, and every product and every sum is rounded to the input dtype
// before the next op.  For bfloat16 this is "compute in fp32, round to bf16"
// per op (bf16*bf16 products are exact in fp32, so only the explicit roundings
// matter).  For float32 the ops are kept separate (no FMA contraction).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace kf {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

enum DType : int { F32 = 0, BF16 = 1, F16 = 2 };

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float x) { return (_Float16)x; }

// Round a float to the storage type and back (the value a T tensor would hold).
template <typename T> __device__ __forceinline__ float round_to(float x) {
  return to_f32(from_f32<T>(x));
}

// Half-split RoPE of one (x1, x2) pair with table values (c, s) given in fp32
// (the reference's float32 tables); eager-op rounding in dtype T.
//   r1 = x1*c - x2*s ; r2 = x2*c + x1*s      (kempnerforge/model/position.py:71)
template <typename T>
__device__ __forceinline__ void rope_pair(float x1, float x2, float cf, float sf,
                                          float& r1, float& r2) {
#pragma clang fp contract(off)
  const float c = round_to<T>(cf);
  const float s = round_to<T>(sf);
  const float a = round_to<T>(x1 * c);
  const float b = round_to<T>(x2 * s);
  const float e = round_to<T>(x2 * c);
  const float f = round_to<T>(x1 * s);
  r1 = round_to<T>(a - b);
  r2 = round_to<T>(e + f);
}

// RoPE backward for one pair (transposed rotation), fp32 in and out; the table
// values are the dtype-cast ones the forward multiplied by.
template <typename T>
__device__ __forceinline__ void rope_pair_bwd(float g1, float g2, float cf, float sf,
                                              float& d1, float& d2) {
  const float c = round_to<T>(cf);
  const float s = round_to<T>(sf);
  d1 = g1 * c + g2 * s;
  d2 = g2 * c - g1 * s;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- 16-bit element types of the MFMA kernels ------------------------------
// The MFMA kernels move bf16 and fp16 tensors as raw 16-bit words (u32x4
// chunks, and bf16x8 vectors as the container of an 8-element MFMA operand
// whatever its type); the element type T (bf16 or f16) decides only how
// those words are converted to and from float and which MFMA multiplies them.
typedef _Float16 f16;
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Two floats -> two round-to-nearest-even T in one dword (lo in bits 0-15).
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  static_assert(std::is_same<T, bf16>::value || std::is_same<T, f16>::value, "16-bit T");
  const f32x2 f = {lo, hi};
  if constexpr (std::is_same<T, bf16>::value)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2));
}
// The two T of a dword as floats (exact).
template <typename T>
__device__ __forceinline__ void unpack2(uint32_t w, float& lo, float& hi) {
  if constexpr (std::is_same<T, bf16>::value) {
    lo = __uint_as_float(w << 16);
    hi = __uint_as_float(w & 0xffff0000u);
  } else {
    const f16x2 h = __builtin_bit_cast(f16x2, w);
    lo = (float)h[0];
    hi = (float)h[1];
  }
}
// Unpack 8 T held in a 16-byte vector into floats.
template <typename T>
__device__ __forceinline__ void unpack8(const u32x4& u, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) unpack2<T>(u[i], f[2 * i], f[2 * i + 1]);
}
template <typename T>
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 u;
#pragma unroll
  for (int i = 0; i < 4; ++i) u[i] = pack2<T>(f[2 * i], f[2 * i + 1]);
  return u;
}

// Round two floats to T (round to nearest even) with one conversion, back to
// fp32: the same bits as two round_to<T>.
template <typename T>
__device__ __forceinline__ void round2(float& x, float& y) {
  unpack2<T>(pack2<T>(x, y), x, y);
}

// rope_pair<T> on 8 pairs, outputs packed as 8 T (r1 -> o1, r2 -> o2).  The
// same bits as rope_pair<T> then pack8, with two roundings per conversion
// instruction and the last rounding done by the pack itself.
template <typename T>
__device__ __forceinline__ void rope8(const float* x1, const float* x2, const float* cf,
                                      const float* sf, u32x4& o1, u32x4& o2) {
#pragma clang fp contract(off)
  float r1[8], r2[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float c = cf[j], s = sf[j];
    round2<T>(c, s);
    float a = x1[j] * c, e = x2[j] * c;
    round2<T>(a, e);
    float b = x2[j] * s, f = x1[j] * s;
    round2<T>(b, f);
    r1[j] = a - b;
    r2[j] = e + f;
  }
  o1 = pack8<T>(r1);
  o2 = pack8<T>(r2);
}

// C += A·B on 32x32x16 (resp. 16x16x32) tiles of T, fp32 accumulation; the
// operands are 8 T each, carried in bf16x8 containers.
template <typename T>
__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  if constexpr (std::is_same<T, bf16>::value)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
template <typename T>
__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  if constexpr (std::is_same<T, bf16>::value)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// DType code of a 16-bit element type (the C ABI's dtype argument).
template <typename T> constexpr int dtype_code();
template <> constexpr int dtype_code<bf16>() { return BF16; }
template <> constexpr int dtype_code<f16>() { return F16; }

}  // namespace kf

// ---------------------------------------------------------------- host side
namespace kf {
void set_error(const char* fmt, ...);
namespace prof {
bool enabled();
void begin(const char* name, hipStream_t s);
void end(hipStream_t s);
}  // namespace prof
}  // namespace kf

// Launch a kernel; with kf_prof_enable(1) the launch is bracketed by HIP events
// on `stream` and attributed to `name`.
#define KF_LAUNCH(name, kernel, grid, block, shmem, stream, ...)          \
  do {                                                                   \
    const bool kf_prof_on_ = kf::prof::enabled();                        \
    if (kf_prof_on_) kf::prof::begin(name, stream);                      \
    hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__); \
    if (kf_prof_on_) kf::prof::end(stream);                              \
  } while (0)

#define KF_CHECK_ARG(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      kf::set_error(__VA_ARGS__);        \
      return KF_ERR_INVALID_ARGUMENT;    \
    }                                    \
  } while (0)

#define KF_CHECK_LAUNCH()                                              \
  do {                                                                 \
    hipError_t e_ = hipGetLastError();                                 \
    if (e_ != hipSuccess) {                                            \
      kf::set_error("kernel launch failed: %s", hipGetErrorString(e_)); \
      return KF_ERR_HIP;                                               \
    }                                                                  \
  } while (0)
