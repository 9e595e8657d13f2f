// SwiGLU forward / backward fused with quantisation:
//   fm_swiglu_quantize      -- h = silu(g) * u from bf16 g, u (one [M, 2H]
//                              buffer or two tensors), emitted as bf16 or e4m3
//                              with row and/or transposed block scales
//   fm_swiglu_backward      -- [dg | du] from one read of g, u and dh, emitted
//                              the same way (the [M, 2H] layout feeds the fused
//                              dx = dg w1 + du w3 GEMM and the dW1|dW3 GEMM)
// silu(g) = g * s, s = sigmoid(g) = 1 / (1 + 2^(-g log2 e)) from the hardware
// v_exp_f32 and v_rcp_f32 (a few fp32 ulps; test_gpu_swiglu.py holds the
// results to torch's CPU silu and autograd); d silu = s (1 + g (1 - s)).
#include "fm_tile.h"
#include "../../include/fm_hip.h"

namespace fm {

__device__ __forceinline__ float sigmoidf(float g) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f));
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
    float gv[8], uv[8];
    unpack8_bf16(r.g, gv);
    unpack8_bf16(r.u, uv);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[0][i] = (gv[i] * sigmoidf(gv[i])) * uv[i];
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
    float gv[8], uv[8], dv[8];
    unpack8_bf16(r.g, gv);
    unpack8_bf16(r.u, uv);
    unpack8_bf16(r.dh, dv);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float s = sigmoidf(gv[i]);
      v[0][i] = dv[i] * uv[i] * s * (1.f + gv[i] * (1.f - s));
      v[1][i] = dv[i] * (gv[i] * s);
    }
  }
};

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

}  // extern "C"
