// SwiGLU forward / backward fused with quantisation:
//   fm_swiglu_quantize      -- h = silu(g) * u from bf16 g, u (one [M, 2H]
//                              buffer or two tensors), emitted as bf16 or e4m3
//                              with row and/or transposed block scales
//   fm_swiglu_backward      -- [dg | du] from one read of g, u and dh, emitted
//                              the same way (the [M, 2H] layout feeds the fused
//                              dx = dg w1 + du w3 GEMM and the dW1|dW3 GEMM)
// silu(g) = g / (1 + e^-g) and d silu = s (1 + g (1 - s)), s = 1 / (1 + e^-g),
// in the reference's (torch's) order of operations; test_gpu_swiglu.py holds
// the results to within 2 ulp of torch's CPU silu and autograd.
#include "fm_tile.h"
#include "../../include/fm_hip.h"

namespace fm {

// e^-g to about an ulp: 2^(-g log2 e) with the product split into a rounded
// part and its exact remainder (the remainder's share of the exponent would
// otherwise cost |g| 2^-24 ln 2 relative), the hardware 2^x on the fraction
// of the rounded part plus the remainder (|x| <= 0.5 + 2^-24), and the integer
// part as an exponent.  Overflow (g < -88.7) gives +inf, which the callers
// treat as IEEE division would.
__device__ __forceinline__ float exp_neg(float g) {
#pragma clang fp contract(off)   // ph must be rounded: pl is its exact remainder
  constexpr float kL = 1.44269502162933349609375f;   // RN(log2 e)
  constexpr float kLlo = 1.925963033500011e-08f;     // log2 e - kL
  const float ph = -g * kL;
  const float pl = fmaf(-g, kLlo, fmaf(-g, kL, -ph));
  const float n = __builtin_rintf(ph);   // 2^x on x in [-0.5, 0.5], then the exponent
  return __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f((ph - n) + pl), int(n));
}

// silu(g) = g / d and sigmoid(g) = 1 / d, d = 1 + e^-g: the expressions of
// the reference's torch silu and its backward (x / (1 + exp(-x)), sigmoid =
// 1 / (1 + exp(-x))).  Quotients from the hardware reciprocal with a
// residual correction (within an ulp of the rounded quotient).  d infinite
// (g < -88.7): sigmoid 0 and silu -0, as IEEE division gives.
__device__ __forceinline__ float silu_only(float g) {
#pragma clang fp contract(off)
  const float d = 1.f + exp_neg(g);
  const float r = __builtin_amdgcn_rcpf(d);
  const float q0 = g * r;
  const float q = fmaf(fmaf(-d, q0, g), r, q0);
  return d <= 3.40282347e38f ? q : g * 0.f;
}

struct SigSilu {
  float s, silu;
};
__device__ __forceinline__ SigSilu sig_silu(float g) {
#pragma clang fp contract(off)
  const float d = 1.f + exp_neg(g);
  float r = __builtin_amdgcn_rcpf(d);
  r = fmaf(fmaf(-d, r, 1.f), r, r);
  const float q0 = g * r;
  const float q = fmaf(fmaf(-d, q0, g), r, q0);
  const bool fin = d <= 3.40282347e38f;
  return SigSilu{fin ? r : 0.f, fin ? q : g * 0.f};
}

struct SwigluSrc {
  static constexpr int kOut = 1;
  const uint16_t* g;  // [M, H] pitch ld_g
  const uint16_t* u;  // [M, H] pitch ld_u
  int64_t ld_g, ld_u;
  struct Raw {
    uint4 g, u;
  };
  __device__ __forceinline__ Raw fetch(int64_t row, int64_t col) const {
    return Raw{*reinterpret_cast<const uint4*>(g + row * ld_g + col),
               *reinterpret_cast<const uint4*>(u + row * ld_u + col)};
  }
  __device__ __forceinline__ void compute(const Raw& r, float v[][8]) const {
#pragma clang fp contract(off)   // every product rounded: the same values in every kernel that inlines this
    float gv[8], uv[8];
    unpack8_bf16(r.g, gv);
    unpack8_bf16(r.u, uv);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[0][i] = silu_only(gv[i]) * uv[i];
  }
};

// Two values per element from one read of g, u, dh: v[0] = dg (output columns
// [0, H)), v[1] = du (output columns [H, 2H)).
struct SwigluBwdSrc {
  static constexpr int kOut = 2;
  const uint16_t* g;
  const uint16_t* u;
  const uint16_t* dh;
  int64_t ld_g, ld_u, ld_dh;
  struct Raw {
    uint4 g, u, dh;
  };
  __device__ __forceinline__ Raw fetch(int64_t row, int64_t col) const {
    return Raw{*reinterpret_cast<const uint4*>(g + row * ld_g + col),
               *reinterpret_cast<const uint4*>(u + row * ld_u + col),
               *reinterpret_cast<const uint4*>(dh + row * ld_dh + col)};
  }
  __device__ __forceinline__ void compute(const Raw& r, float v[][8]) const {
#pragma clang fp contract(off)   // every product and sum rounded, as in the other kernels inlining this
    float gv[8], uv[8], dv[8];
    unpack8_bf16(r.g, gv);
    unpack8_bf16(r.u, uv);
    unpack8_bf16(r.dh, dv);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // torch autograd of silu(g) * u: dy = dh * u, dg = dy * s * (1 + g (1 - s)),
      // du = dh * silu(g), each operation rounded in this order
      const SigSilu ss = sig_silu(gv[i]);
      v[0][i] = ((dv[i] * uv[i]) * ss.s) * (1.f + gv[i] * (1.f - ss.s));
      v[1][i] = dv[i] * ss.silu;
    }
  }
};

// The fp32 values a source hands to the tile producer, written out as they
// are (one thread per 8 columns of a row): what the fused quantisers round.
template <typename Src>
__global__ __launch_bounds__(256) void source_values_kernel(Src src, int64_t rows, int64_t cols, float* out,
                                                            int64_t ld_out, int64_t col_off1) {
  const int64_t chunks = cols / 8;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < rows * chunks; i += int64_t(gridDim.x) * 256) {
    const int64_t r = i / chunks, c = (i % chunks) * 8;
    float v[Src::kOut][8];
    src.compute(src.fetch(r, c), v);
#pragma unroll
    for (int o = 0; o < Src::kOut; ++o) {
      float* p = out + r * ld_out + c + o * col_off1;
      *reinterpret_cast<float4*>(p) = make_float4(v[o][0], v[o][1], v[o][2], v[o][3]);
      *reinterpret_cast<float4*>(p + 4) = make_float4(v[o][4], v[o][5], v[o][6], v[o][7]);
    }
  }
}

}  // namespace fm

using namespace fm;

extern "C" {

int fm_swiglu_quantize(const void* g, int64_t ld_g, const void* u, int64_t ld_u, int64_t rows,
                       int64_t H, int kind, void* q, int64_t ld_q, void* s, int64_t ld_s, void* qt,
                       int64_t ld_qt, void* st, int64_t ld_st, const int32_t* tile_valid,
                       void* stream) {
  FM_REQUIRE((g && u) || rows == 0, "fm_swiglu_quantize: null input");
  FM_REQUIRE(ld_g % 8 == 0 && ld_u % 8 == 0 && ld_g >= H && ld_u >= H,
             "fm_swiglu_quantize: pitches must be multiples of 8 and >= H");
  const TileOut o = make_tile_out(kind, q, ld_q, s, ld_s, qt, ld_qt, st, ld_st, 0, 0, tile_valid);
  SwigluSrc src{static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(u), ld_g, ld_u};
  return launch_tile_producer(src, o, rows, H, static_cast<hipStream_t>(stream),
                              "fm_swiglu_quantize");
}

int fm_swiglu_backward(const void* g, int64_t ld_g, const void* u, int64_t ld_u, const void* dh,
                       int64_t ld_dh, int64_t rows, int64_t H, int kind, void* q, int64_t ld_q,
                       void* s, int64_t ld_s, void* qt, int64_t ld_qt, void* st, int64_t ld_st,
                       const int32_t* tile_valid, void* stream) {
  FM_REQUIRE((g && u && dh) || rows == 0, "fm_swiglu_backward: null input");
  FM_REQUIRE(H % 128 == 0, "fm_swiglu_backward: H must be a multiple of 128");
  FM_REQUIRE(ld_g % 8 == 0 && ld_u % 8 == 0 && ld_dh % 8 == 0,
             "fm_swiglu_backward: pitches must be multiples of 8");
  const TileOut o = make_tile_out(kind, q, ld_q, s, ld_s, qt, ld_qt, st, ld_st, 0, H, tile_valid);
  SwigluBwdSrc src{static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(u),
                   static_cast<const uint16_t*>(dh), ld_g, ld_u, ld_dh};
  return launch_tile_producer(src, o, rows, H, static_cast<hipStream_t>(stream),
                              "fm_swiglu_backward");
}

int fm_swiglu_values(const void* g, int64_t ld_g, const void* u, int64_t ld_u, const void* dh, int64_t ld_dh,
                     int64_t rows, int64_t H, float* out, int64_t ld_out, void* stream) {
  FM_REQUIRE((g && u && out) || rows == 0, "fm_swiglu_values: null pointer");
  FM_REQUIRE(H % 8 == 0 && ld_g % 8 == 0 && ld_u % 8 == 0 && (dh == nullptr || ld_dh % 8 == 0),
             "fm_swiglu_values: H and pitches must be multiples of 8");
  FM_REQUIRE(ld_out % 4 == 0 && ld_out >= (dh ? 2 * H : H), "fm_swiglu_values: output pitch too small");
  if (rows == 0) return 0;
  const int64_t n = rows * (H / 8);
  const unsigned blocks = unsigned(n / 256 + 1 < 16384 ? n / 256 + 1 : 16384);
  hipStream_t sm = static_cast<hipStream_t>(stream);
  if (dh) {
    SwigluBwdSrc src{static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(u),
                     static_cast<const uint16_t*>(dh), ld_g, ld_u, ld_dh};
    hipLaunchKernelGGL(source_values_kernel<SwigluBwdSrc>, dim3(blocks), dim3(256), 0, sm, src, rows, H, out,
                       ld_out, H);
  } else {
    SwigluSrc src{static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(u), ld_g, ld_u};
    hipLaunchKernelGGL(source_values_kernel<SwigluSrc>, dim3(blocks), dim3(256), 0, sm, src, rows, H, out,
                       ld_out, 0);
  }
  return check_launch("fm_swiglu_values");
}

}  // extern "C"
