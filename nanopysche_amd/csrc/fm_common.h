// Device helpers shared by the fp8_flow_moe HIP kernels (gfx950 / CDNA4).
//
// Number formats:
//   bf16   -- stored as uint16_t; widened by a 16-bit shift, narrowed with
//             round-to-nearest-even.
//   e4m3   -- OCP e4m3fn (bias 7, max 448, 0x7F/0xFF NaN, no infinities).
//             f32 -> e4m3 is an integer round-to-nearest-even routine; it is
//             __host__ __device__ so the host test build can check it against
//             torch's cast exhaustively.
//   e8m0   -- OCP MX shared exponent, value 2^(code-127).
//
// Block-scale spec (blockwise recipes):
//   amax  = max |x| over the block (fp32)
//   scale = max(amax, 1e-12f) / 448.0f             (IEEE fp32 division)
//   pow2 recipe: scale = 2^ceil(log2(scale))       (exponent-field round up)
//   q     = e4m3(clamp(x / scale, -448, 448))
// MX spec (1x32): code = clamp(biased_exp(amax) - 8, 0, 254),
//   q = e4m3_saturate(x * 2^(127-code)).
#pragma once

#include <stdint.h>
#include <atomic>
#include <hip/hip_runtime.h>

#define FM_HD __host__ __device__ __forceinline__

namespace fm {

constexpr float kE4M3Max = 448.0f;
constexpr float kAmaxFloor = 1e-12f;
constexpr int kBlock = 128;
constexpr int kMxBlock = 32;

FM_HD uint32_t f2u(float f) { union { float f; uint32_t u; } v; v.f = f; return v.u; }
FM_HD float u2f(uint32_t u) { union { float f; uint32_t u; } v; v.u = u; return v.f; }

FM_HD float bf16_to_f32(uint16_t b) { return u2f(uint32_t(b) << 16); }

FM_HD uint16_t f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

// f32 -> e4m3fn, round-to-nearest-even, non-saturating (|x| > 464 -> NaN).
// Callers clamp to +-448 first, so the NaN branch only sees NaN inputs.
FM_HD uint8_t f32_to_e4m3(float x) {
  uint32_t u = f2u(x);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x43e80000u) return uint8_t(sign | 0x7fu);   // > 464 or NaN / inf
  if (a < 0x3c800000u) {                               // < 2^-6: e4m3 subnormal
    // value = m * 2^-9, m = RNE(|x| * 2^9) in [0, 8]; 8 is the smallest normal
    float s = u2f(a) * 512.0f;                         // exact (power of two)
    uint32_t m = uint32_t(s);                          // truncate
    float frac = s - float(m);
    if (frac > 0.5f || (frac == 0.5f && (m & 1u))) m += 1u;
    return uint8_t(sign | m);
  }
  // normal: keep 3 mantissa bits, round the dropped 20 bits to nearest-even;
  // a carry out of the mantissa bumps the exponent, which is the right answer.
  uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
  uint32_t code = (r >> 20) - (120u << 3);             // rebias 127 -> 7
  if (code > 0x7eu) code = 0x7eu;                      // 448 < x <= 464 -> 448
  return uint8_t(sign | code);
}

FM_HD float e4m3_to_f32(uint8_t c) {
  uint32_t sign = uint32_t(c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xfu, m = c & 7u;
  if ((c & 0x7fu) == 0x7fu) return u2f(sign | 0x7fc00000u);
  if (e == 0) return u2f(sign | f2u(float(m) * 0.001953125f));  // m * 2^-9
  return u2f(sign | ((e + 120u) << 23) | (m << 20));
}

FM_HD float clamp448(float v) { return fminf(fmaxf(v, -kE4M3Max), kE4M3Max); }

// Blockwise scale from the block's amax.
FM_HD float block_scale(float amax, bool pow2) {
  float s = fmaxf(amax, kAmaxFloor) / kE4M3Max;
  if (pow2) {
    uint32_t u = f2u(s);
    uint32_t e = (u >> 23) & 0xffu;
    if (u & 0x7fffffu) e += 1u;
    s = u2f(e << 23);
  }
  return s;
}

FM_HD uint8_t quant_e4m3(float x, float scale) { return f32_to_e4m3(clamp448(x / scale)); }

// Stores to device buffers through global-memory pointers.  A store through
// a pointer the compiler cannot place in global memory (one built from an
// integer, or loaded from LDS) is a FLAT store, which counts in lgkmcnt as well
// as vmcnt: every later wait for an LDS access then also waits for the store to
// reach memory, and the vmcnt waits for later loads become full drains.
// (HIP's vector types are classes whose assignment is declared for generic
// objects only, so the stores go through clang's native vectors.)
typedef uint32_t fm_u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t fm_u32x4 __attribute__((ext_vector_type(4)));
typedef float fm_f32x4 __attribute__((ext_vector_type(4)));
#define FM_GLOBAL(T, p) ((__attribute__((address_space(1))) T*)(p))
__device__ __forceinline__ void st_global(void* p, uint4 v) { *FM_GLOBAL(fm_u32x4, p) = fm_u32x4{v.x, v.y, v.z, v.w}; }
__device__ __forceinline__ void st_global(void* p, uint2 v) { *FM_GLOBAL(fm_u32x2, p) = fm_u32x2{v.x, v.y}; }
__device__ __forceinline__ void st_global(void* p, float4 v) { *FM_GLOBAL(fm_f32x4, p) = fm_f32x4{v.x, v.y, v.z, v.w}; }
__device__ __forceinline__ void st_global(float* p, float v) { *FM_GLOBAL(float, p) = v; }
__device__ __forceinline__ void st_global(uint8_t* p, uint8_t v) { *FM_GLOBAL(uint8_t, p) = v; }
__device__ __forceinline__ void st_global(uint16_t* p, uint16_t v) { *FM_GLOBAL(uint16_t, p) = v; }
__device__ __forceinline__ void st_global(uint32_t* p, uint32_t v) { *FM_GLOBAL(uint32_t, p) = v; }

// gfx950 v_cvt_pk_fp8_f32 (OCP e4m3fn, round-to-nearest-even) on four values
// already clamped to +-448; byte i of the result encodes value i.  The GPU test
// test_gpu_quant.py::test_hw_convert_matches_software checks it against the
// integer routine above.
__device__ __forceinline__ uint32_t hw_e4m3x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __builtin_bit_cast(int, a), false);  // high half set below
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return uint32_t(w);
}
// gfx950 v_cvt_pk_f32_fp8 on the four e4m3 bytes of w (byte i -> f[i]); exact.
// test_gpu_quant.py::test_hw_decode_matches_software checks all 256 codes.
__device__ __forceinline__ void hw_dec_e4m3x4(uint32_t w, float f[4]) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8(int(w), false);
  const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8(int(w), true);
  f[0] = lo[0];
  f[1] = lo[1];
  f[2] = hi[0];
  f[3] = hi[1];
}
// x / s rounded to nearest for the quotients a block quantiser forms
// (|x| <= 448 s up to rounding, or s infinite), from a reciprocal computed once
// per block: y = RN(1/s), q0 = RN(x y), e = q0 s - x (exact, one FMA),
// q = RN(q0 - e y) is the correctly rounded quotient whenever it is a normal
// number (Markstein, IBM J. Res. Dev. 34(1), 1990); below the normal range it
// can differ, and such quotients encode to e4m3 zero either way.  The
// correction multiplies by ny = -y rather than negating e, so a zero x keeps
// its sign (e = +0, e * ny = -0).  For an infinite s the correction uses 0 in
// place of s, so q = x * 0, as x / s.
struct Recip {
  float sd;  // s, or 0 when s is infinite
  float ny;  // -RN(1 / s)
};
__device__ __forceinline__ Recip recip_of(float s) { return Recip{s <= 3.40282347e38f ? s : 0.f, -(1.0f / s)}; }
__device__ __forceinline__ float div_rn(float x, Recip d) {
  const float q0 = x * -d.ny;
  const float e = fmaf(q0, d.sd, -x);
  return fmaf(e, d.ny, q0);
}
// a / 448 rounded to nearest for a >= 1e-12 (the amax floor), in three
// operations: the Markstein correction with the constant RN(1/448) gives the
// correctly rounded quotient for every finite a in that range (checked
// exhaustively on the CPU against IEEE division); an infinite a is returned.
__device__ __forceinline__ float div448(float a) {
  constexpr float y = 1.0f / kE4M3Max;
  const float q0 = a * y;
  const float r = fmaf(q0, -kE4M3Max, a);
  const float q = fmaf(r, y, q0);
  return a <= 3.40282347e38f ? q : a;
}
// block_scale on the device, with div448 for the division.
__device__ __forceinline__ float block_scale_dev(float amax, bool pow2) {
  float s = div448(fmaxf(amax, kAmaxFloor));
  if (pow2) {
    uint32_t u = f2u(s);
    uint32_t e = (u >> 23) & 0xffu;
    if (u & 0x7fffffu) e += 1u;
    s = u2f(e << 23);
  }
  return s;
}
// 1 / s for a power-of-two scale s = 2^k, k in [-126, 126], from the exponent
// field (exact); 0 for an infinite s.
__device__ __forceinline__ float pow2_recip(float s) {
  const uint32_t e = (f2u(s) >> 23) & 0xffu;
  return e == 0xffu ? 0.f : u2f((254u - e) << 23);
}
// clamp to +-448 in one v_med3_f32 (equal to clamp448 for every non-NaN value)
__device__ __forceinline__ float clamp448_med3(float v) {
  return __builtin_amdgcn_fmed3f(v, -kE4M3Max, kE4M3Max);
}
// gfx950 v_cvt_pk_bf16_f32 (round-to-nearest-even): low half = a.
__device__ __forceinline__ uint32_t hw_bf16x2(float a, float b) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  const bf2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// MX shared-exponent code of a block with this amax.
FM_HD uint32_t mx_code(float amax) {
  int e = int((f2u(amax) >> 23) & 0xffu) - 8;
  e = e < 0 ? 0 : (e > 254 ? 254 : e);
  return uint32_t(e);
}
// 2^(127 - code) as a float (code in [0, 254] -> exponent field 254 - code).
FM_HD float mx_inv_scale(uint32_t code) {
  uint32_t f = 254u - code;
  return f == 0u ? u2f(0x00400000u) : u2f(f << 23);
}
FM_HD float e8m0_to_f32(uint32_t code) {
  return code == 0u ? u2f(0x00400000u) : u2f(code << 23);
}
FM_HD uint8_t quant_mx(float x, float inv_scale) { return f32_to_e4m3(clamp448(x * inv_scale)); }

}  // namespace fm

// ----------------------------------------------------------- error plumbing ----
// Every C-ABI entry point returns 0 on success or a nonzero code; the message
// of the last failure on the calling thread is kept for fm_last_error_string.
namespace fm {
void set_error(const char* fmt, ...);
int check_launch(const char* what);

// Compute units of the current device (cached per device).
inline int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// A null pointer or one on a 16-byte boundary (the vector accesses' alignment).
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Workgroups of `kernel` (`block` threads, no dynamic LDS) that fit on the
// device at once: its occupancy per CU (registers, LDS) x the CUs.  A launch
// of that many workgroups runs in one round, with no partly filled last one.
template <typename F>
inline int64_t resident_workgroups(F kernel, int block) {
  int nb = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel, block, 0) != hipSuccess || nb < 1) nb = 1;
  return int64_t(nb) * device_cus();
}
}  // namespace fm

#define FM_REQUIRE(cond, ...)            \
  do {                                   \
    if (!(cond)) {                       \
      fm::set_error(__VA_ARGS__);        \
      return 1;                          \
    }                                    \
  } while (0)
