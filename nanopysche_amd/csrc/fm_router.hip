// Router gate of the MoE layer (reference MoERouter.forward, model/moe.py:133-184):
//   fm_router_forward    the whole forward of the router in two launches for small gates
//                        (E <= 8, D = 512 n <= 2048): logits, top-k gating, the softmax
//                        and logsumexp^2 partials and per-workgroup expert histograms in
//                        one pass over x, then counts + load-balancing (+ z) loss; other
//                        shapes run the same steps as separate kernels
//   fm_router_logits     logits[t][e] = sum_d x[t][d] * w[e][d] + bias[e] + score_bias[e], fp32
//                        (the reference's gate(x.float()) + score_bias, :151-154)
//   fm_expert_counts     counts[e] = number of the T*K slots routed to e (the f_i of the
//                        load-balancing loss, :267-281)
//   fm_gating_grad       dlogits from the gradient of the top-k weights (softmax over the K
//                        selected logits, :249-255, or normalised sigmoid, :257-265) plus the
//                        gradient of the load-balancing loss E * sum_i f_i P_i;
//                        fm_gating_grad_dot forms the weights' gradient itself from the
//                        expert outputs, <dout[t], y[row(t, k)]>, in the same pass
//   fm_router_backward   dx = dlogits w, dw = dlogits^T x, db = sum_t dlogits (fp32 sums in a
//                        fixed order: per-slice partials in a caller workspace, then the
//                        slices in order), dw and db written in the parameters' dtype
//
// The gate is a skinny GEMM (E <= 256 outputs per token): x is read once at
// its size and the products are summed in fp32, as the reference computes
// it -- on the matrix cores for bf16 x and a bf16 gate with E <= 8, D <= 2048
// (bf16 products are exact in fp32; the order of the sums differs), otherwise
// as FMAs on the VALU; HBM, not arithmetic, bounds it at the layer's shapes.
// Gate weights are read as stored (fp32 or bf16).
#include <type_traits>

#include "fm_gating.h"
#include "../../include/fm_hip.h"

namespace fm {

constexpr int kRouterRows = 16;    // token rows per workgroup (4 waves x 4 rows)
constexpr int kRouterCols = 512;   // d-columns per chunk (64 lanes x 8)

__device__ __forceinline__ void load8f(const uint16_t* p, float (&v)[8]) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = u2f(w[j] << 16);
    v[2 * j + 1] = u2f(w[j] & 0xffff0000u);
  }
}
__device__ __forceinline__ void load8f(const float* p, float (&v)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
__device__ __forceinline__ void store8(uint16_t* p, const float (&v)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    w[j] = uint32_t(f32_to_bf16(v[2 * j])) | (uint32_t(f32_to_bf16(v[2 * j + 1])) << 16);
  *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
}
__device__ __forceinline__ void store8(float* p, const float (&v)[8]) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Gate weights are read as stored (fp32, or bf16 widened exactly), so the
// fp32 arithmetic sees the parameter's own values with no conversion pass.
__device__ __forceinline__ float4 ldw4(const void* w, int bf16, int64_t i) {
  if (bf16) {
    const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(w) + i);
    return make_float4(u2f(u.x << 16), u2f(u.x & 0xffff0000u), u2f(u.y << 16), u2f(u.y & 0xffff0000u));
  }
  return *reinterpret_cast<const float4*>(static_cast<const float*>(w) + i);
}
__device__ __forceinline__ float ldw1(const void* w, int bf16, int64_t i) {
  return bf16 ? bf16_to_f32(static_cast<const uint16_t*>(w)[i]) : static_cast<const float*>(w)[i];
}

// Stages w[e0 .. e0+EC)[c0 .. c0+kRouterCols) into LDS (zero past E or D).
// All of a thread's loads are issued before its LDS stores (a fixed trip
// count), so staging costs one memory latency, not one per element group.
template <int EC>
__device__ __forceinline__ void stage_gate(float (&wl)[EC][kRouterCols], const void* w, int w_bf16, int64_t ld_w,
                                           int E, int64_t D, int e0, int64_t c0) {
  constexpr int kPer = EC * kRouterCols / 4 / 256;
  float4 v[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int i = threadIdx.x + 256 * u;
    const int e = i / (kRouterCols / 4), c = (i % (kRouterCols / 4)) * 4;
    v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e0 + e < E && c0 + c < D) v[u] = ldw4(w, w_bf16, (e0 + e) * ld_w + c0 + c);
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int i = threadIdx.x + 256 * u;
    *reinterpret_cast<float4*>(&wl[i / (kRouterCols / 4)][(i % (kRouterCols / 4)) * 4]) = v[u];
  }
}

// ------------------------------------------------------------ forward ----
struct RouterArgs {
  const void* x;
  int64_t ld_x, T, D;
  const void* w;          // [E, ld_w] fp32 or bf16 (w_bf16)
  int64_t ld_w;
  const void* bias;       // [E], the weight's dtype, or null
  int w_bf16;
  const float* score_bias;
  int E;
  float* logits;
  int64_t ld_l;
};

// grid (T / 16, ceil(E / EC)); wave v owns rows 16*blockIdx.x + 4v .. +4, lane l
// columns 8l .. 8l+8 of each 512-column chunk; sums over the 64 lanes at the end.
template <typename T, int EC>
__global__ __launch_bounds__(256) void router_logits_kernel(RouterArgs a) {
  __shared__ __attribute__((aligned(16))) float wl[EC][kRouterCols];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = int64_t(blockIdx.x) * kRouterRows + wave * 4;
  const int e0 = blockIdx.y * EC;
  const T* x = static_cast<const T*>(a.x);
  float acc[4][EC];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int e = 0; e < EC; ++e) acc[r][e] = 0.f;
  for (int64_t c0 = 0; c0 < a.D; c0 += kRouterCols) {
    __syncthreads();
    stage_gate<EC>(wl, a.w, a.w_bf16, a.ld_w, a.E, a.D, e0, c0);
    __syncthreads();
    const int64_t col = c0 + lane * 8;
    if (col < a.D) {
      float xv[4][8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (r0 + r < a.T) {
          load8f(x + (r0 + r) * a.ld_x + col, xv[r]);
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) xv[r][j] = 0.f;
        }
      }
#pragma unroll
      for (int e = 0; e < EC; ++e) {
        const float4 w0 = *reinterpret_cast<const float4*>(&wl[e][lane * 8]);
        const float4 w1 = *reinterpret_cast<const float4*>(&wl[e][lane * 8 + 4]);
        const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[r][e] = fmaf(xv[r][j], wv[j], acc[r][e]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int e = 0; e < EC; ++e) {
      const float s = wave_sum(acc[r][e]);
      const int eg = e0 + e;
      if (lane == e && eg < a.E && r0 + r < a.T) {
        float v = s;
        if (a.bias) v += ldw1(a.bias, a.w_bf16, eg);
        if (a.score_bias) v += a.score_bias[eg];
        a.logits[(r0 + r) * a.ld_l + eg] = v;
      }
    }
}

// Small gates (E <= 8, D <= 2048, D % 512 == 0): the whole gate sits in LDS (dynamic, 8 D
// floats, at most 64 KiB: two workgroups per CU), staged once, and each wave
// walks its 4 rows over D with the next 512-column chunk of x already in
// flight (no barrier inside the loop).
constexpr int kGateLdsBytes = 64 * 1024;

// Sum of v[i] over the 64 lanes for 32 values per lane as a reduce-scatter:
// each exchange halves the values a lane keeps (32 shuffles in all, against
// 32 x 6 for separate wave sums); lane l ends with the total of value l / 2.
// The lane's choice between v[i] and v[i + half] is made on the bits with a
// mask: written as `up ? v[i] : v[i + half]` the compiler turned it into
// v[i + (up ? 0 : half)], a runtime index into the 32 registers, i.e.
// compare/select chains over all of them (~3300 instructions per call).
__device__ __forceinline__ float wave_reduce_scatter32(float (&v)[32], int lane) {
#pragma unroll
  for (int l = 0; l < 5; ++l) {
    const int o = 32 >> l, half = 16 >> l;
    const uint32_t m = (lane & o) != 0 ? 0xffffffffu : 0u;   // up: send the low half
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (i < half) {
        const uint32_t lo = __float_as_uint(v[i]), hi = __float_as_uint(v[i + half]);
        const float send = __uint_as_float((lo & m) | (hi & ~m));
        const float keep = __uint_as_float((hi & m) | (lo & ~m));
        v[i] = keep + __shfl_xor(send, o);
      }
    }
  }
  return v[0] + __shfl_xor(v[0], 1);
}

template <typename T>
__device__ __forceinline__ void load8_row(const T* row, int64_t col, float (&v)[8]) {
  load8f(row + col, v);
}

__device__ __forceinline__ void bf16x8_to_f32(const uint4 u, float (&v)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = u2f(w[j] << 16);
    v[2 * j + 1] = u2f(w[j] & 0xffff0000u);
  }
}

// acc[row][expert] += x chunk (8 values of each of 4 rows) . gate chunk
// acc[row][expert] += x chunk (8 values of each of 4 rows) . gate chunk; the
// gate in LDS as fp32 or as the bf16 it was stored in (widened here, exactly)
template <typename WL>
__device__ __forceinline__ void router_fma_chunk(float (&acc)[32], const float (&xv)[4][8], const WL* wc,
                                                 int64_t D) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float wv[8];
    if constexpr (sizeof(WL) == 2) {
      bf16x8_to_f32(*reinterpret_cast<const uint4*>(wc + e * D), wv);
    } else {
      const float4 w0 = *reinterpret_cast<const float4*>(wc + e * D);
      const float4 w1 = *reinterpret_cast<const float4*>(wc + e * D + 4);
      wv[0] = w0.x; wv[1] = w0.y; wv[2] = w0.z; wv[3] = w0.w;
      wv[4] = w1.x; wv[5] = w1.y; wv[6] = w1.z; wv[7] = w1.w;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[r * 8 + e] = fmaf(xv[r][j], wv[j], acc[r * 8 + e]);
  }
}

// With FUSED the same workgroup also gates its 16 tokens (gate_group, the
// gating kernel's per-token code, on the logits it just formed), writes the
// per-wave softmax / logsumexp^2 partials of the load-balancing and z losses,
// and its expert histogram of the routed slots (router_finish_kernel turns
// those into counts and the loss).
struct RouterFuse {
  GateOut go;
  float* prob_partial;   // [E, gridDim.x]: per-workgroup softmax sums (waves 0..3 in order)
  float* z_partial;      // [gridDim.x] or null
  int32_t* block_hist;   // [E, gridDim.x]
};

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// bf16 x and gate, D <= 2048: the workgroup's 16 x 8 logits as one 16x16
// MFMA tile (tokens x experts, experts 8..15 zero), wave w contracting its
// quarter of D (at most 16 steps of 32: x and gate fragments loaded straight
// into registers, the gate from L2), then the four partial tiles summed
// through LDS in a fixed order.  Products of bf16 values are exact in the
// fp32 accumulator; only the summation order differs from the VALU path.
// Returns this lane's logit of the VALU path's layout: token 4 wave + (lane
// / 16), expert (lane / 2) % 8.
__device__ __forceinline__ float router_logits_mfma(const RouterArgs& a, int lane, int wave,
                                                    float (&red)[4][16][17]) {
  const int kq = int(a.D / 4);   // a multiple of 128
  const int nm = kq / 32;        // <= 16
  const int64_t row = int64_t(blockIdx.x) * kRouterRows + (lane & 15);
  const uint16_t* xr = static_cast<const uint16_t*>(a.x) + (row < a.T ? row : a.T - 1) * a.ld_x;
  const int en = lane & 15;
  const bool ev = en < a.E;
  const uint16_t* wr = static_cast<const uint16_t*>(a.w) + int64_t(ev ? en : 0) * a.ld_w;
  const int k0 = wave * kq + 8 * (lane >> 4);
  uint4 xa[16], wb[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    if (m < nm) {
      xa[m] = *reinterpret_cast<const uint4*>(xr + k0 + 32 * m);
      wb[m] = ev ? *reinterpret_cast<const uint4*>(wr + k0 + 32 * m) : make_uint4(0, 0, 0, 0);
    }
  }
  v4f c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < 16; ++m)
    if (m < nm)
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, xa[m]), __builtin_bit_cast(v8bf, wb[m]),
                                                  c, 0, 0, 0);
  // lane l holds tile rows (tokens) 4 (l / 16) + i, column (expert) l % 16
#pragma unroll
  for (int i = 0; i < 4; ++i) red[wave][4 * (lane >> 4) + i][en] = c[i];
  __syncthreads();
  const int vi = lane >> 1, tr = 4 * wave + (vi >> 3), e = vi & 7;
  return ((red[0][tr][e] + red[1][tr][e]) + red[2][tr][e]) + red[3][tr][e];
}

template <typename T, typename WL, bool FUSED>
__global__ __launch_bounds__(256) void router_logits_small_kernel(RouterArgs a, RouterFuse f) {
  extern __shared__ __attribute__((aligned(16))) uint4 wl_raw[];
  WL* wl = reinterpret_cast<WL*>(wl_raw);   // [8][D]: fp32, or the bf16 gate as stored
  __shared__ int32_t hist[8];
  __shared__ float wpart[4][9];   // per wave: softmax sums of experts 0..7, logsumexp^2
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (FUSED && threadIdx.x < 8) hist[threadIdx.x] = 0;
  const int64_t r0 = int64_t(blockIdx.x) * kRouterRows + wave * 4;
  const int64_t D = a.D;
  const int nc = int(D / kRouterCols);   // D % 512 == 0 (launcher)
  // bf16 x and gate, D <= 2048: the logits on the matrix cores; otherwise
  // (an fp32 input or gate, or a longer row) fp32 FMAs on the VALU
  constexpr bool kMfma = sizeof(T) == 2 && sizeof(WL) == 2;
  float sum;
  if (kMfma && nc <= 4) {
    __shared__ float red[4][16][17];
    sum = router_logits_mfma(a, lane, wave, red);
  } else {
    // rows past T re-read the last row (their sums are not stored)
    const T* rows[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = r0 + r < a.T ? r0 + r : a.T - 1;
      rows[r] = static_cast<const T*>(a.x) + row * a.ld_x + lane * 8;
    }
    // bf16 rows of at most 2048 columns: all of this wave's x loads are issued
    // right after the gate's loads and before the gate's LDS stores, so the
    // stores wait only for the gate (loads complete in issue order) and the two
    // memory latencies overlap; the chunk loop then waits on none
    constexpr bool kWhole = sizeof(T) == 2;
    const bool whole = kWhole && nc <= 4;
    uint4 xr[4][4];
    auto load_x = [&]() {
      if (whole) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (c < nc) xr[c][r] = *reinterpret_cast<const uint4*>(rows[r] + int64_t(c) * kRouterCols);
      }
    };
    if constexpr (sizeof(WL) == 2) {
      // the bf16 gate copied as stored: 8 rows of D <= 4096 over 256 threads, at
      // most two 16-byte pieces per thread and row, all loads before the stores
      constexpr int kPerRow = kGateLdsBytes / 8 / 16 / 256;
      uint4 v[8][kPerRow];
      const int Di = int(D);
      const uint16_t* w = static_cast<const uint16_t*>(a.w);
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int u = 0; u < kPerRow; ++u) {
          const int c = (int(threadIdx.x) + 256 * u) * 8;
          v[e][u] = make_uint4(0, 0, 0, 0);
          if (c < Di && e < a.E) v[e][u] = *reinterpret_cast<const uint4*>(w + e * a.ld_w + c);
        }
      load_x();
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int u = 0; u < kPerRow; ++u) {
          const int c = (int(threadIdx.x) + 256 * u) * 8;
          if (c < Di) *reinterpret_cast<uint4*>(&wl[e * Di + c]) = v[e][u];
        }
    } else {
      // 8 gate rows of D <= 2048 floats over 256 threads: per row at most two
      // float4 per thread (expert x column loop, no index division), all loads
      // issued before the stores
      constexpr int kPerRow = kGateLdsBytes / 4 / 8 / 1024;
      float4 v[8][kPerRow];
      const int Di = int(D);
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int u = 0; u < kPerRow; ++u) {
          const int c = (int(threadIdx.x) + 256 * u) * 4;
          v[e][u] = make_float4(0.f, 0.f, 0.f, 0.f);
          if (c < Di && e < a.E) v[e][u] = ldw4(a.w, a.w_bf16, e * a.ld_w + c);
        }
      load_x();
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int u = 0; u < kPerRow; ++u) {
          const int c = (int(threadIdx.x) + 256 * u) * 4;
          if (c < Di) *reinterpret_cast<float4*>(&wl[e * Di + c]) = v[e][u];
        }
    }
    __syncthreads();
    float acc[32];   // [row][expert]
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] = 0.f;
    if (whole) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (c < nc) {
          float xv[4][8];
#pragma unroll
          for (int r = 0; r < 4; ++r) bf16x8_to_f32(xr[c][r], xv[r]);
          router_fma_chunk(acc, xv, wl + int64_t(c) * kRouterCols + lane * 8, D);
        }
      }
    } else {
      float cur[4][8], nxt[4][8];
#pragma unroll
      for (int r = 0; r < 4; ++r) load8f(rows[r], cur[r]);
      for (int c = 0; c < nc; ++c) {
        const int cn = c + 1 < nc ? c + 1 : c;
#pragma unroll
        for (int r = 0; r < 4; ++r) load8f(rows[r] + int64_t(cn) * kRouterCols, nxt[r]);
        router_fma_chunk(acc, cur, wl + int64_t(c) * kRouterCols + lane * 8, D);
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int j = 0; j < 8; ++j) cur[r][j] = nxt[r][j];
      }
    }
    sum = wave_reduce_scatter32(acc, lane);
  }
  const int vi = lane >> 1, r = vi >> 3, e = vi & 7;
  float lv = sum;
  if (e < a.E) {
    if (a.bias) lv += ldw1(a.bias, a.w_bf16, e);
    if (a.score_bias) lv += a.score_bias[e];
  }
  if ((lane & 1) == 0 && e < a.E && r0 + r < a.T) a.logits[(r0 + r) * a.ld_l + e] = lv;
  if constexpr (FUSED) {
    // token slot g = lane / 8 (tokens r0 .. r0 + 3; slots 4..7 idle), expert lane % 8
    const int g = lane >> 3, ge = lane & 7;
    const float lg = __shfl(lv, 2 * (8 * (g & 3) + ge));
    const int64_t t = r0 + g;
    const bool tv = g < 4 && t < a.T;
    float psum = 0.f, zsum = 0.f;
    const int my_i = gate_group<8>(f.go, t, tv, g, ge, (tv && ge < a.E) ? lg : -INFINITY, psum, zsum);
    if (tv && ge < f.go.K) atomicAdd(&hist[my_i], 1);
#pragma unroll
    for (int off = 8; off < 64; off <<= 1) psum += __shfl_xor(psum, off);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) zsum += __shfl_xor(zsum, off);
    if (lane < 8) wpart[wave][lane] = psum;
    if (lane == 0) wpart[wave][8] = zsum;
    __syncthreads();
    const int64_t nb = gridDim.x;
    if (threadIdx.x < a.E) {
      const int e = threadIdx.x;
      f.block_hist[e * nb + blockIdx.x] = hist[e];
      f.prob_partial[e * nb + blockIdx.x] = ((wpart[0][e] + wpart[1][e]) + wpart[2][e]) + wpart[3][e];
    }
    if (f.z_partial && threadIdx.x == 0)
      f.z_partial[blockIdx.x] = ((wpart[0][8] + wpart[1][8]) + wpart[2][8]) + wpart[3][8];
  }
}

// Counts and loss after the fused router forward (one workgroup: wave e < E
// per expert, wave 8 for the z-loss): counts[e] = sum of the workgroups'
// histograms (exact), optionally added to the running totals; loss = E *
// sum_e (counts_e / T) (P_e / T) with P_e the sum of the per-workgroup softmax
// partials, plus z_mult * (sum of the logsumexp^2 partials) / T.  Each wave
// sums its contiguous row of partials in lane-strided runs of eight loads,
// then a fixed shuffle tree.
__global__ __launch_bounds__(576) void router_finish_kernel(const int32_t* block_hist, int64_t nb, int E,
                                                            int32_t* counts, int64_t* acc, int64_t* acc_total,
                                                            int64_t T, const float* prob_partial,
                                                            const float* z_partial, float z_mult, float* loss) {
  __shared__ float term[8];
  __shared__ float zterm;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool zw = wave == 8;
  if (wave < E || (zw && z_partial)) {
    const int32_t* hrow = block_hist + int64_t(wave) * nb;
    const float* prow = zw ? z_partial : prob_partial + int64_t(wave) * nb;
    int c = 0;
    float p = 0.f;
    for (int64_t b0 = 0; b0 < nb; b0 += 512) {
      int cv[8];
      float pv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t b = b0 + u * 64 + lane;
        cv[u] = (!zw && b < nb) ? hrow[b] : 0;
        pv[u] = b < nb ? prow[b] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        c += cv[u];
        p += pv[u];
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      c += __shfl_xor(c, off);
      p += __shfl_xor(p, off);
    }
    if (lane == 0) {
      if (zw) {
        zterm = p / float(T);
      } else {
        counts[wave] = c;
        if (acc) acc[wave] += c;
        term[wave] = (float(c) / float(T)) * (p / float(T));
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    if (acc_total) acc_total[0] += T;
    float sum = 0.f;
    for (int e = 0; e < E; ++e) sum += term[e];
    float l = float(E) * sum;
    if (z_partial) l = l + z_mult * zterm;
    loss[0] = l;
  }
}

// --------------------------------------------------------------- counts ----
// One workgroup: LDS histogram over all T*K slots (fixed E <= 1024 bins).
// With `acc` the counts are also added to the running per-expert totals and
// `tokens` to acc_total (the workgroup owns them: no atomics).
template <typename I>
__global__ __launch_bounds__(1024) void expert_counts_kernel(const I* idx, int64_t n, int E, int32_t* counts,
                                                             int64_t* acc, int64_t* acc_total, int64_t tokens) {
  __shared__ int32_t h[1024];
  for (int e = threadIdx.x; e < E; e += 1024) h[e] = 0;
  __syncthreads();
  for (int64_t i = threadIdx.x; i < n; i += 1024) {
    const int64_t e = int64_t(idx[i]);
    if (e >= 0 && e < E) atomicAdd(&h[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 1024) {
    counts[e] = h[e];
    if (acc) acc[e] += h[e];
  }
  if (acc && threadIdx.x == 0) acc_total[0] += tokens;
}

// post_batch: score_bias[e] += gamma * (acc[e] / total - 1 / E) in fp32, then
// the running totals are cleared; nothing happens while total is 0.
__global__ __launch_bounds__(1024) void score_bias_update_kernel(int64_t* acc, int64_t* acc_total, int E,
                                                                 float gamma, float* score_bias) {
#pragma clang fp contract(off)   // separately rounded multiply and add, as the reference's tensor ops
  const int64_t total = acc_total[0];
  __syncthreads();   // every thread has read the total before thread 0 clears it
  if (total == 0) return;
  const float ideal = 1.0f / float(E);
  for (int e = threadIdx.x; e < E; e += 1024) {
    const float actual = float(acc[e]) / float(total);
    score_bias[e] = score_bias[e] + gamma * (actual - ideal);
    acc[e] = 0;
  }
  if (threadIdx.x == 0) acc_total[0] = 0;
}

// ---------------------------------------------------------- gating grad ----
struct GatingGradArgs {
  const float* logits;   // [T, ld_l]
  int64_t T, ld_l;
  int E, K;
  int sigmoid;           // sigmoid weights (0: softmax over the selected logits, also for replay)
  int l2;                // the forward divided the weights by their l2 norm + 1e-8
  const void* idx;       // [T, K]
  int idx_i64;
  const float* dw;       // [T, K] or null
  const float* daux;     // scalar or null
  const int32_t* counts; // [E] (needed with daux)
  float z_mult;          // z-loss multiplier (0: no z-loss)
  float* dlogits;        // [T, ld_d]
  int64_t ld_d;
  // the weights' gradient formed here instead of read from dw (DOT kernels):
  // dw[t, k] = <dout[t], y[row_of[t K + k]]> (0 for a dropped slot, row -1)
  const uint16_t* dout;  // bf16 [T, ld_do]
  int64_t ld_do;
  const uint16_t* y;     // bf16 [rows, ld_y]
  int64_t ld_y;
  const int32_t* row_of; // [T K]
  int64_t D;
  float* dw_out;         // [T, K] or null: the formed weights' gradient
};

constexpr int kDotMaxK = 8;

// dots[k] (every lane) = <dout[t], y[row_of[t K + k]]> for k < K <= KD: lane
// l takes columns 8 l .. of each 512-column chunk; a pass over CH chunks
// issues all of its dout and y loads before the FMAs (8 / KD chunks, so at
// most nine 16-byte loads per lane wait at once); the K partial sums meet in
// a wave sum each.
template <int KD>
__device__ __forceinline__ void slot_dots(const GatingGradArgs& a, int64_t t, int lane, float (&dots)[kDotMaxK]) {
  constexpr int CH = KD >= 8 ? 1 : 8 / KD;
  int rk[KD];
#pragma unroll
  for (int k = 0; k < kDotMaxK; ++k) dots[k] = 0.f;
#pragma unroll
  for (int k = 0; k < KD; ++k) rk[k] = k < a.K ? a.row_of[t * a.K + k] : -1;
  const uint16_t* g = a.dout + t * a.ld_do;
  for (int64_t c0 = 0; c0 < a.D; c0 += 512 * CH) {
    uint4 gr[CH], yr[KD][CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int64_t col = c0 + 512 * c + lane * 8;
      const bool cv = col < a.D;
      gr[c] = cv ? *reinterpret_cast<const uint4*>(g + col) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int k = 0; k < KD; ++k)
        yr[k][c] = (cv && rk[k] >= 0) ? *reinterpret_cast<const uint4*>(a.y + int64_t(rk[k]) * a.ld_y + col)
                                      : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      float gv[8];
      bf16x8_to_f32(gr[c], gv);
#pragma unroll
      for (int k = 0; k < KD; ++k) {
        float yv[8];
        bf16x8_to_f32(yr[k][c], yv);
#pragma unroll
        for (int j = 0; j < 8; ++j) dots[k] += gv[j] * yv[j];
      }
    }
  }
#pragma unroll
  for (int k = 0; k < KD; ++k)
    if (k < a.K) dots[k] = wave_sum(dots[k]);
}

constexpr int kGateMaxPerLane = 4;  // E <= 256

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// One wave per token (grid-stride); lane holds experts lane + 64 j, and lane
// k < K also slot k of the token.  The weights before the optional l2
// normalisation are recomputed from the logits:
//   softmax (and R3 replay): u_k = softmax over the K selected logits
//   sigmoid:                 u_k = s_k / (S + 1e-8), S = sum_k s_k
// l2: w = u / (n + 1e-8), n = ||u||, so du = dw / (n + 1e-8) - u (u.dw) / (n (n + 1e-8)^2).
// Then c = sum_k u_k du_k and expert i_k gets
//   softmax: u_k (du_k - c);  sigmoid: (du_k - c) / (S + 1e-8) * s_k (1 - s_k).
template <int KD>   // KD > 0: the weights' gradient formed here, K <= KD
__global__ __launch_bounds__(256) void gating_grad_kernel(GatingGradArgs a) {
  constexpr bool DOT = KD > 0;
  const int lane = threadIdx.x & 63;
  const int64_t n_waves = int64_t(gridDim.x) * 4;
  const float aux = a.daux ? a.daux[0] : 0.f;
  for (int64_t t = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6); t < a.T; t += n_waves) {
    float v[kGateMaxPerLane], g[kGateMaxPerLane];
#pragma unroll
    for (int j = 0; j < kGateMaxPerLane; ++j) {
      const int e = lane + 64 * j;
      v[j] = e < a.E ? a.logits[t * a.ld_l + e] : -INFINITY;
      g[j] = 0.f;
    }
    if (DOT || a.dw) {
      float mine = 0.f;
      if constexpr (DOT) {
        float dots[kDotMaxK];
        slot_dots<KD>(a, t, lane, dots);
#pragma unroll
        for (int k = 0; k < kDotMaxK; ++k) mine = lane == k ? dots[k] : mine;
        if (a.dw_out && lane < a.K) a.dw_out[int64_t(t) * a.K + lane] = mine;
      }
      // slots outside [0, E) carry no weight and no gradient
      int ik = -1;
      float lk = -INFINITY, dk = 0.f;
      if (lane < a.K) {
        const int64_t i = int64_t(t) * a.K + lane;
        ik = a.idx_i64 ? int(static_cast<const int64_t*>(a.idx)[i]) : static_cast<const int32_t*>(a.idx)[i];
        if (ik >= 0 && ik < a.E) {
          lk = a.logits[t * a.ld_l + ik];
          dk = DOT ? mine : a.dw[i];
        } else {
          ik = -1;
        }
      }
      float u, S = 0.f, sk = 0.f;
      if (a.sigmoid) {
        sk = ik >= 0 ? 1.f / (1.f + expf(-lk)) : 0.f;
        S = wave_sum(sk);
        u = sk / (S + 1e-8f);
      } else {
        const float mk = wave_max(lk);
        const float ek = ik >= 0 ? expf(lk - mk) : 0.f;
        u = ek / wave_sum(ek);
      }
      float du = dk;
      if (a.l2) {
        const float n = sqrtf(wave_sum(u * u));
        const float dot = wave_sum(u * dk);
        const float ne = n + 1e-8f;
        du = dk / ne - (n > 0.f ? u * dot / (n * ne * ne) : 0.f);
      }
      const float c = wave_sum(u * du);
      const float gk = ik < 0 ? 0.f
                              : (a.sigmoid ? (du - c) / (S + 1e-8f) * sk * (1.f - sk) : u * (du - c));
      for (int k = 0; k < a.K; ++k) {
        const int ek = __shfl(ik, k);
        const float gv = __shfl(gk, k);
        if (ek >= 0 && (ek & 63) == lane) {
#pragma unroll
          for (int j = 0; j < kGateMaxPerLane; ++j)
            if ((ek >> 6) == j) g[j] += gv;
        }
      }
    }
    // load-balancing loss: d/dl_e = daux * (E / T) * p_e * (f_e - sum_j f_j p_j),
    // p = softmax over all E, f_e = counts_e / T; z-loss (mean over tokens of
    // logsumexp^2): d/dl_e = daux * z_mult * (2 / T) * lse * p_e
    if (a.daux) {
      float m = -INFINITY;
#pragma unroll
      for (int j = 0; j < kGateMaxPerLane; ++j) m = fmaxf(m, v[j]);
      m = wave_max(m);
      float p[kGateMaxPerLane], f[kGateMaxPerLane], s = 0.f;
#pragma unroll
      for (int j = 0; j < kGateMaxPerLane; ++j) {
        const int e = lane + 64 * j;
        p[j] = e < a.E ? expf(v[j] - m) : 0.f;
        f[j] = e < a.E ? float(a.counts[e]) / float(a.T) : 0.f;
        s += p[j];
      }
      s = wave_sum(s);
      float fp = 0.f;
#pragma unroll
      for (int j = 0; j < kGateMaxPerLane; ++j) {
        p[j] /= s;
        fp += f[j] * p[j];
      }
      fp = wave_sum(fp);
      const float scale = aux * float(a.E) / float(a.T);
      const float zs = a.z_mult != 0.f ? aux * a.z_mult * 2.f * (m + logf(s)) / float(a.T) : 0.f;
#pragma unroll
      for (int j = 0; j < kGateMaxPerLane; ++j) g[j] += scale * p[j] * (f[j] - fp) + zs * p[j];
    }
#pragma unroll
    for (int j = 0; j < kGateMaxPerLane; ++j) {
      const int e = lane + 64 * j;
      if (e < a.E) a.dlogits[t * a.ld_d + e] = g[j];
    }
  }
}

// ------------------------------------------------------------- backward ----
struct RouterBwdArgs {
  const float* dl;       // [T, ld_dl]
  int64_t ld_dl;
  const void* x;         // [T, ld_x]
  int64_t ld_x, T, D;
  const void* w;         // [E, ld_w], fp32 or bf16 (w_bf16)
  int64_t ld_w;
  int w_bf16;
  int E;
  void* dx;              // [T, ld_dx], x's dtype (null: skip)
  int64_t ld_dx;
  float* part;           // [slices][E][D] partial dw
  float* part_db;        // [slices][E] partial db, or null
  int64_t slices, rows_per_slice;
};

// dx: grid (T / 16); wave v rows 16 b + 4 v .. +4, lane l columns 8 l .. of
// each 512-column chunk, sum over all experts in chunks of 16.
template <typename T>
__global__ __launch_bounds__(256) void router_dx_kernel(RouterBwdArgs a) {
  __shared__ __attribute__((aligned(16))) float wl[16][kRouterCols];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = int64_t(blockIdx.x) * kRouterRows + wave * 4;
  T* dx = static_cast<T*>(a.dx);
  for (int64_t c0 = 0; c0 < a.D; c0 += kRouterCols) {
    const int64_t col = c0 + lane * 8;
    float acc[4][8];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[r][j] = 0.f;
    for (int e0 = 0; e0 < a.E; e0 += 16) {
      __syncthreads();
      stage_gate<16>(wl, a.w, a.w_bf16, a.ld_w, a.E, a.D, e0, c0);
      __syncthreads();
      if (col < a.D) {
#pragma unroll 4
        for (int e = 0; e < 16 && e0 + e < a.E; ++e) {
          const float4 w0 = *reinterpret_cast<const float4*>(&wl[e][lane * 8]);
          const float4 w1 = *reinterpret_cast<const float4*>(&wl[e][lane * 8 + 4]);
          const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float d = r0 + r < a.T ? a.dl[(r0 + r) * a.ld_dl + e0 + e] : 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[r][j] = fmaf(d, wv[j], acc[r][j]);
          }
        }
      }
    }
    if (col < a.D) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (r0 + r < a.T) store8(dx + (r0 + r) * a.ld_dx + col, acc[r]);
    }
  }
}

// Partial dw: grid (ceil(D / 256), slices, ceil(E / 8)); the slice's rows are
// split over the 4 waves (row t of the slice to wave t % 4), lane l owns
// columns 4 l .. 4 l + 3 of the workgroup's 256 for 8 experts (narrow
// columns: twice the workgroups for the same partials).  Each wave issues
// the loads of eight of its rows before their FMAs (row order kept): x stays
// packed in registers, and the dlogits of a row -- the same for every lane --
// come as two 16-byte loads of a wave-uniform address.  The 4 waves' sums meet
// in one 4 KiB LDS buffer in wave order (wave 0 writes, waves 1, 2, 3 add).
// The workgroups of column block 0 also form the slice's db partial (each
// wave's rows in order, then waves 0..3).
constexpr int kDwCols = 256;

template <typename T>
__global__ __launch_bounds__(256) void router_dw_kernel(RouterBwdArgs a) {
  constexpr int EG = 8, RB = 8;
  __shared__ __attribute__((aligned(16))) float red[EG][kDwCols];
  __shared__ float dbred[4][EG];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int64_t col = int64_t(blockIdx.x) * kDwCols + lane * 4;
  const int64_t s = blockIdx.y;
  const int e0 = blockIdx.z * EG;
  const bool want_db = a.part_db != nullptr && blockIdx.x == 0;
  const int64_t t_lo = s * a.rows_per_slice;
  const int64_t t_hi = t_lo + a.rows_per_slice < a.T ? t_lo + a.rows_per_slice : a.T;
  const T* x = static_cast<const T*>(a.x);
  const bool cv = col < a.D;
  const int64_t cl = cv ? col : 0;   // rows are read in full; columns past D are not stored
  const bool full8 = e0 + EG <= a.E && a.ld_dl % 4 == 0;
  using Raw = typename std::conditional<sizeof(T) == 2, uint2, float4>::type;
  float acc[EG][4], dbacc[EG];
#pragma unroll
  for (int e = 0; e < EG; ++e) {
    dbacc[e] = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[e][j] = 0.f;
  }
  auto dl_row = [&](int64_t t, float (&d)[EG]) {
    const float* p = a.dl + t * a.ld_dl + e0;
    if (full8) {
      const float4 v0 = *reinterpret_cast<const float4*>(p);
      const float4 v1 = *reinterpret_cast<const float4*>(p + 4);
      d[0] = v0.x; d[1] = v0.y; d[2] = v0.z; d[3] = v0.w;
      d[4] = v1.x; d[5] = v1.y; d[6] = v1.z; d[7] = v1.w;
    } else {
#pragma unroll
      for (int e = 0; e < EG; ++e) d[e] = e0 + e < a.E ? p[e] : 0.f;
    }
  };
  auto widen4 = [](const Raw& r, float (&v)[4]) {
    if constexpr (sizeof(T) == 2) {
      const uint2 u = *reinterpret_cast<const uint2*>(&r);
      v[0] = u2f(u.x << 16); v[1] = u2f(u.x & 0xffff0000u);
      v[2] = u2f(u.y << 16); v[3] = u2f(u.y & 0xffff0000u);
    } else {
      const float4 f = *reinterpret_cast<const float4*>(&r);
      v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    }
  };
  auto row_fma = [&](const float (&xv)[4], const float (&d)[EG]) {
#pragma unroll
    for (int e = 0; e < EG; ++e) {
      dbacc[e] += d[e];
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[e][j] = fmaf(d[e], xv[j], acc[e][j]);
    }
  };
  int64_t t = t_lo + wave;
  for (; t + 4 * (RB - 1) < t_hi; t += 4 * RB) {
    Raw xr[RB];
    float dv[RB][EG];
#pragma unroll
    for (int u = 0; u < RB; ++u) {
      xr[u] = *reinterpret_cast<const Raw*>(x + (t + 4 * u) * a.ld_x + cl);
      dl_row(t + 4 * u, dv[u]);
    }
#pragma unroll
    for (int u = 0; u < RB; ++u) {
      float xv[4];
      widen4(xr[u], xv);
      row_fma(xv, dv[u]);
    }
  }
  for (; t < t_hi; t += 4) {
    float xv[4], d[EG];
    widen4(*reinterpret_cast<const Raw*>(x + t * a.ld_x + cl), xv);
    dl_row(t, d);
    row_fma(xv, d);
  }
  if (want_db && lane == 0)
#pragma unroll
    for (int e = 0; e < EG; ++e) dbred[wave][e] = dbacc[e];
  // ((w0 + w1) + w2) + w3 through one buffer
  for (int w = 0; w < 4; ++w) {
    if (wave == w) {
#pragma unroll
      for (int e = 0; e < EG; ++e) {
        float4* p = reinterpret_cast<float4*>(&red[e][lane * 4]);
        float4 q = w == 0 ? make_float4(0.f, 0.f, 0.f, 0.f) : *p;
        if (w == 0) q = make_float4(acc[e][0], acc[e][1], acc[e][2], acc[e][3]);
        else { q.x += acc[e][0]; q.y += acc[e][1]; q.z += acc[e][2]; q.w += acc[e][3]; }
        *p = q;
      }
    }
    __syncthreads();
  }
  for (int i = threadIdx.x; i < EG * kDwCols / 4; i += 256) {
    const int e = i / (kDwCols / 4), c = (i % (kDwCols / 4)) * 4;
    const int64_t gc = int64_t(blockIdx.x) * kDwCols + c;
    if (e0 + e < a.E && gc < a.D)
      *reinterpret_cast<float4*>(a.part + (s * a.E + e0 + e) * a.D + gc) =
          *reinterpret_cast<const float4*>(&red[e][c]);
  }
  if (want_db && threadIdx.x < EG && e0 + int(threadIdx.x) < a.E) {
    const int e = threadIdx.x;
    a.part_db[s * a.E + e0 + e] = ((dbred[0][e] + dbred[1][e]) + dbred[2][e]) + dbred[3][e];
  }
}

// dw[e][d] = sum over the slices of the partials: a workgroup owns 64
// elements, wave q sums slices q, q + 4, ... (eight loads in flight), and the
// four wave sums are added in wave order.  The last workgroup forms db the
// same way per expert (lane-strided slices, then a fixed shuffle tree).  Both
// are written as fp32 or bf16.
__global__ __launch_bounds__(256) void router_dw_reduce_kernel(RouterBwdArgs a, void* dw, int64_t ld_dw, int dw_bf16,
                                                               void* db, int db_bf16) {
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int64_t n = int64_t(a.E) * a.D;
  if (blockIdx.x == gridDim.x - 1) {
    if (db == nullptr) return;
    for (int e = q; e < a.E; e += 4) {
      float v = 0.f;
#pragma unroll 8
      for (int64_t sl = lane; sl < a.slices; sl += 64) v += a.part_db[sl * a.E + e];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
      if (lane == 0) {
        if (db_bf16) static_cast<uint16_t*>(db)[e] = f32_to_bf16(v);
        else static_cast<float*>(db)[e] = v;
      }
    }
    return;
  }
  if (dw == nullptr) return;
  const int64_t i = int64_t(blockIdx.x) * 64 + lane;
  float v = 0.f;
  if (i < n) {
#pragma unroll 8
    for (int64_t sl = q; sl < a.slices; sl += 4) v += a.part[sl * n + i];
  }
  red[q][lane] = v;
  __syncthreads();
  if (q == 0 && i < n) {
    const float t = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
    const int64_t o = (i / a.D) * ld_dw + i % a.D;
    if (dw_bf16) static_cast<uint16_t*>(dw)[o] = f32_to_bf16(t);
    else static_cast<float*>(dw)[o] = t;
  }
}

// The fused forward takes the small-gate kernel's shapes; others fall back to
// separate kernels (their gating uses this many waves of partials).
constexpr int64_t kRouterForwardWaves = 1024;

// the small-gate kernel: E <= 8, D = 512 n, the gate [8, D] in at most 64 KiB of LDS (fp32: D <= 2048;
// a bf16 gate stays bf16: D <= 4096)
inline bool router_small_ok(int E, int64_t D, int w_bf16) {
  return E <= 8 && D % kRouterCols == 0 && 8 * D * (w_bf16 ? 2 : 4) <= kGateLdsBytes;
}

int router_logits_launch(const RouterArgs& a, int x_dtype, const RouterFuse* f, int fused, hipStream_t s,
                         const char* what) {
  const unsigned rb = unsigned((a.T + kRouterRows - 1) / kRouterRows);
  const bool xb = x_dtype == FM_DTYPE_BF16;
  if (router_small_ok(a.E, a.D, a.w_bf16)) {
    const size_t lds = size_t(8 * a.D) * (a.w_bf16 ? 2 : 4);
    const RouterFuse none{};
    const RouterFuse& ff = f ? *f : none;
    const dim3 g(rb), b(256);
#define FM_SMALL(XT, WL, FU) hipLaunchKernelGGL((router_logits_small_kernel<XT, WL, FU>), g, b, lds, s, a, ff)
    if (fused) {
      if (a.w_bf16) { if (xb) FM_SMALL(uint16_t, uint16_t, true); else FM_SMALL(float, uint16_t, true); }
      else { if (xb) FM_SMALL(uint16_t, float, true); else FM_SMALL(float, float, true); }
    } else {
      if (a.w_bf16) { if (xb) FM_SMALL(uint16_t, uint16_t, false); else FM_SMALL(float, uint16_t, false); }
      else { if (xb) FM_SMALL(uint16_t, float, false); else FM_SMALL(float, float, false); }
    }
#undef FM_SMALL
  } else if (a.E <= 8) {
    const dim3 grid(rb, 1);
    if (xb) hipLaunchKernelGGL((router_logits_kernel<uint16_t, 8>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((router_logits_kernel<float, 8>), grid, dim3(256), 0, s, a);
  } else {
    const dim3 grid(rb, unsigned((a.E + 15) / 16));
    if (xb) hipLaunchKernelGGL((router_logits_kernel<uint16_t, 16>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((router_logits_kernel<float, 16>), grid, dim3(256), 0, s, a);
  }
  return check_launch(what);
}

// slices of the token range for the dw partials: at most 128, and at most
// 32 MiB of partials
inline int64_t router_slices(int64_t T, int64_t D, int E) {
  int64_t s = (32ll << 20) / (int64_t(E) * D * 4);
  s = s < 128 ? s : 128;
  s = s < 1 ? 1 : s;
  const int64_t per = (T + s - 1) / s;
  return per > 0 ? (T + per - 1) / per : 1;
}

}  // namespace fm

using namespace fm;

extern "C" {

int fm_router_logits(const void* x, int x_dtype, int64_t ld_x, int64_t T, int64_t D, const void* w, int w_dtype,
                     int64_t ld_w, const void* bias, const float* score_bias, int E, float* logits, int64_t ld_l,
                     void* stream) {
  FM_REQUIRE(x && w && logits, "fm_router_logits: null pointer");
  FM_REQUIRE(x_dtype == FM_DTYPE_BF16 || x_dtype == FM_DTYPE_F32, "fm_router_logits: bad x dtype %d", x_dtype);
  FM_REQUIRE(w_dtype == FM_DTYPE_BF16 || w_dtype == FM_DTYPE_F32, "fm_router_logits: bad gate dtype %d", w_dtype);
  FM_REQUIRE(E >= 1 && E <= 256, "fm_router_logits: E must be in [1, 256] (got %d)", E);
  FM_REQUIRE(D > 0 && D % 8 == 0, "fm_router_logits: D must be a positive multiple of 8 (got %lld)", (long long)D);
  FM_REQUIRE(ld_x >= D && ld_x % 8 == 0 && ld_w >= D && ld_w % 4 == 0 && ld_l >= E,
             "fm_router_logits: bad pitches");
  if (T == 0) return 0;
  const RouterArgs a{x, ld_x, T, D, w, ld_w, bias, w_dtype == FM_DTYPE_BF16, score_bias, E, logits, ld_l};
  return router_logits_launch(a, x_dtype, nullptr, 0, static_cast<hipStream_t>(stream), "fm_router_logits");
}

int64_t fm_router_forward_workspace_bytes(int64_t T, int E) {
  if (T <= 0 || E <= 0) return 0;
  const int64_t nb = (T + kRouterRows - 1) / kRouterRows;
  const int64_t fused = nb * (int64_t(E) + 1) * 4 + nb * int64_t(E) * 4;
  const int64_t plain = kRouterForwardWaves * (int64_t(E) + 1) * 4;
  return fused > plain ? fused : plain;
}

int fm_router_forward_fused(int E, int64_t D, int w_dtype) {
  return E >= 1 && D > 0 && router_small_ok(E, D, w_dtype == FM_DTYPE_BF16) ? 1 : 0;
}

int fm_router_forward(const void* x, int x_dtype, int64_t ld_x, int64_t T, int64_t D, const void* w, int w_dtype,
                      int64_t ld_w, const void* bias, const float* score_bias, int E, int K, int gating, int flags,
                      const void* replay_indices, int replay_i64, float* logits, int64_t ld_l, float* weights,
                      void* indices, int indices_i64, int32_t* counts, int64_t* tokens_per_expert,
                      int64_t* total_tokens, float z_loss_multiplier, float* loss, void* workspace,
                      int64_t workspace_bytes, void* stream) {
  FM_REQUIRE(x && w && logits && weights && indices && counts && loss, "fm_router_forward: null pointer");
  FM_REQUIRE(x_dtype == FM_DTYPE_BF16 || x_dtype == FM_DTYPE_F32, "fm_router_forward: bad x dtype %d", x_dtype);
  FM_REQUIRE(w_dtype == FM_DTYPE_BF16 || w_dtype == FM_DTYPE_F32, "fm_router_forward: bad gate dtype %d", w_dtype);
  FM_REQUIRE(E >= 1 && E <= 256, "fm_router_forward: E must be in [1, 256] (got %d)", E);
  FM_REQUIRE(K >= 1 && K <= E && K <= 64, "fm_router_forward: K must be in [1, min(E, 64)] (got %d)", K);
  FM_REQUIRE(gating == FM_GATING_SOFTMAX || gating == FM_GATING_SIGMOID, "fm_router_forward: bad gating");
  FM_REQUIRE((flags & ~FM_GATING_L2_NORMALIZE) == 0, "fm_router_forward: unknown flags 0x%x", flags);
  FM_REQUIRE(D > 0 && D % 8 == 0, "fm_router_forward: D must be a positive multiple of 8 (got %lld)", (long long)D);
  FM_REQUIRE(ld_x >= D && ld_x % 8 == 0 && ld_w >= D && ld_w % 4 == 0 && ld_l >= E,
             "fm_router_forward: bad pitches");
  FM_REQUIRE((tokens_per_expert == nullptr) == (total_tokens == nullptr),
             "fm_router_forward: tokens_per_expert and total_tokens go together");
  FM_REQUIRE(T > 0, "fm_router_forward: T must be positive (the loss divides by it)");
  FM_REQUIRE(workspace != nullptr && workspace_bytes >= fm_router_forward_workspace_bytes(T, E),
             "fm_router_forward: workspace of fm_router_forward_workspace_bytes(T, E) bytes required");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const RouterArgs a{x, ld_x, T, D, w, ld_w, bias, w_dtype == FM_DTYPE_BF16, score_bias, E, logits, ld_l};
  const int sigmoid = gating == FM_GATING_SIGMOID;
  const int l2 = (flags & FM_GATING_L2_NORMALIZE) ? 1 : 0;
  const float zm = z_loss_multiplier;
  float* base = static_cast<float*>(workspace);
  if (router_small_ok(E, D, w_dtype == FM_DTYPE_BF16)) {
    const int64_t nb = (T + kRouterRows - 1) / kRouterRows;
    float* part = base;
    float* zpart = base + nb * E;
    int32_t* hist = reinterpret_cast<int32_t*>(zpart + nb);
    const RouterFuse f{GateOut{E, K, sigmoid, l2, replay_indices, replay_i64, weights, indices, indices_i64, 1},
                       part, zm != 0.f ? zpart : nullptr, hist};
    if (int rc = router_logits_launch(a, x_dtype, &f, 1, s, "fm_router_forward")) return rc;
    hipLaunchKernelGGL(router_finish_kernel, dim3(1), dim3(576), 0, s, hist, nb, E, counts, tokens_per_expert,
                       total_tokens, T, part, zm != 0.f ? zpart : nullptr, zm, loss);
    return check_launch("fm_router_forward");
  }
  // other shapes: logits, then gating, counts and loss as separate kernels
  float* part = base;
  float* zpart = base + kRouterForwardWaves * E;
  if (int rc = router_logits_launch(a, x_dtype, nullptr, 0, s, "fm_router_forward")) return rc;
  if (int rc = fm_topk_gating(logits, T, E, ld_l, K, gating, flags, replay_indices, replay_i64, weights, indices,
                              indices_i64, part, zm != 0.f ? zpart : nullptr, kRouterForwardWaves, stream))
    return rc;
  if (int rc = fm_expert_counts(indices, indices_i64, T * K, E, counts, tokens_per_expert, total_tokens, T, stream))
    return rc;
  return fm_aux_loss(part, kRouterForwardWaves, counts, E, T, zm != 0.f ? zpart : nullptr, zm, loss, stream);
}

int fm_expert_counts(const void* indices, int indices_i64, int64_t n, int E, int32_t* counts,
                     int64_t* tokens_per_expert, int64_t* total_tokens, int64_t tokens, void* stream) {
  FM_REQUIRE(indices && counts, "fm_expert_counts: null pointer");
  FM_REQUIRE(E >= 1 && E <= 1024, "fm_expert_counts: E must be in [1, 1024] (got %d)", E);
  FM_REQUIRE(n >= 0 && tokens >= 0, "fm_expert_counts: n and tokens must be >= 0");
  FM_REQUIRE((tokens_per_expert == nullptr) == (total_tokens == nullptr),
             "fm_expert_counts: tokens_per_expert and total_tokens go together");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (indices_i64)
    hipLaunchKernelGGL((expert_counts_kernel<int64_t>), dim3(1), dim3(1024), 0, s,
                       static_cast<const int64_t*>(indices), n, E, counts, tokens_per_expert, total_tokens, tokens);
  else
    hipLaunchKernelGGL((expert_counts_kernel<int32_t>), dim3(1), dim3(1024), 0, s,
                       static_cast<const int32_t*>(indices), n, E, counts, tokens_per_expert, total_tokens, tokens);
  return check_launch("fm_expert_counts");
}

int fm_score_bias_update(int64_t* tokens_per_expert, int64_t* total_tokens, int E, float gamma, float* score_bias,
                         void* stream) {
  FM_REQUIRE(tokens_per_expert && total_tokens && score_bias, "fm_score_bias_update: null pointer");
  FM_REQUIRE(E >= 1 && E <= 1024, "fm_score_bias_update: E must be in [1, 1024] (got %d)", E);
  hipLaunchKernelGGL(score_bias_update_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream),
                     tokens_per_expert, total_tokens, E, gamma, score_bias);
  return check_launch("fm_score_bias_update");
}

int fm_gating_grad(const float* logits, int64_t T, int E, int64_t ld_l, int K, int gating, int flags,
                   int replay, const void* indices, int indices_i64, const float* dweights, const float* daux,
                   const int32_t* counts, float z_loss_multiplier, float* dlogits, int64_t ld_d, void* stream) {
  return fm_gating_grad_dot(logits, T, E, ld_l, K, gating, flags, replay, indices, indices_i64, dweights, nullptr, 0,
                            nullptr, 0, nullptr, 0, nullptr, daux, counts, z_loss_multiplier, dlogits, ld_d, stream);
}

int fm_gating_grad_dot(const float* logits, int64_t T, int E, int64_t ld_l, int K, int gating, int flags, int replay,
                       const void* indices, int indices_i64, const float* dweights, const void* dout, int64_t ld_do,
                       const void* y, int64_t ld_y, const int32_t* row_of, int64_t D, float* dweights_out,
                       const float* daux, const int32_t* counts, float z_loss_multiplier, float* dlogits,
                       int64_t ld_d, void* stream) {
  FM_REQUIRE(logits && indices && dlogits, "fm_gating_grad: null pointer");
  FM_REQUIRE(E >= 1 && E <= 64 * kGateMaxPerLane, "fm_gating_grad: E must be in [1, %d] (got %d)",
             64 * kGateMaxPerLane, E);
  FM_REQUIRE(K >= 1 && K <= E && K <= 64, "fm_gating_grad: K must be in [1, min(E, 64)] (got %d)", K);
  FM_REQUIRE(gating == FM_GATING_SOFTMAX || gating == FM_GATING_SIGMOID, "fm_gating_grad: bad gating");
  FM_REQUIRE((flags & ~FM_GATING_L2_NORMALIZE) == 0, "fm_gating_grad: unknown flags 0x%x", flags);
  FM_REQUIRE(daux == nullptr || counts != nullptr, "fm_gating_grad: the aux-loss gradient needs counts");
  FM_REQUIRE(ld_l >= E && ld_d >= E, "fm_gating_grad: pitch < E");
  const bool dot = dout != nullptr;
  FM_REQUIRE(!dot || (y && row_of && dweights == nullptr), "fm_gating_grad: the fused dot needs y and row_of, "
             "and takes no dweights");
  FM_REQUIRE(!dot || (K <= kDotMaxK && D > 0 && D % 8 == 0 && ld_do >= D && ld_y >= D && ld_do % 8 == 0 &&
                      ld_y % 8 == 0),
             "fm_gating_grad: the fused dot needs K <= %d, D a positive multiple of 8 and pitches >= D (multiples "
             "of 8)", kDotMaxK);
  if (T == 0) return 0;
  const GatingGradArgs a{logits, T, ld_l, E, K, (gating == FM_GATING_SIGMOID && !replay) ? 1 : 0,
                         (flags & FM_GATING_L2_NORMALIZE) ? 1 : 0, indices, indices_i64, dweights, daux,
                         counts, z_loss_multiplier, dlogits, ld_d, static_cast<const uint16_t*>(dout), ld_do,
                         static_cast<const uint16_t*>(y), ld_y, row_of, D, dweights_out};
  const int64_t blocks = (T + 3) / 4 < 4096 ? (T + 3) / 4 : 4096;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid{unsigned(blocks)}, block{256};
  if (!dot) hipLaunchKernelGGL(gating_grad_kernel<0>, grid, block, 0, s, a);
  else if (K <= 2) hipLaunchKernelGGL(gating_grad_kernel<2>, grid, block, 0, s, a);
  else if (K <= 4) hipLaunchKernelGGL(gating_grad_kernel<4>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(gating_grad_kernel<8>, grid, block, 0, s, a);
  return check_launch("fm_gating_grad");
}

int64_t fm_router_workspace_bytes(int64_t T, int64_t D, int E) {
  if (T <= 0 || D <= 0 || E <= 0) return 0;
  return router_slices(T, D, E) * int64_t(E) * (D + 1) * int64_t(sizeof(float));
}

int fm_router_backward(const float* dlogits, int64_t ld_dl, const void* x, int x_dtype, int64_t ld_x, int64_t T,
                       int64_t D, const void* w, int w_dtype, int64_t ld_w, int E, void* dx, int64_t ld_dx, void* dw,
                       int dw_dtype, int64_t ld_dw, void* db, int db_dtype, void* workspace, int64_t workspace_bytes,
                       void* stream) {
  FM_REQUIRE(dlogits && x && (w || dx == nullptr), "fm_router_backward: null pointer");
  FM_REQUIRE(x_dtype == FM_DTYPE_BF16 || x_dtype == FM_DTYPE_F32, "fm_router_backward: bad x dtype %d", x_dtype);
  FM_REQUIRE(w_dtype == FM_DTYPE_BF16 || w_dtype == FM_DTYPE_F32, "fm_router_backward: bad gate dtype %d", w_dtype);
  FM_REQUIRE(dw_dtype == FM_DTYPE_BF16 || dw_dtype == FM_DTYPE_F32, "fm_router_backward: bad dw dtype %d", dw_dtype);
  FM_REQUIRE(db_dtype == FM_DTYPE_BF16 || db_dtype == FM_DTYPE_F32, "fm_router_backward: bad db dtype %d", db_dtype);
  FM_REQUIRE(E >= 1 && E <= 256, "fm_router_backward: E must be in [1, 256] (got %d)", E);
  FM_REQUIRE(D > 0 && D % 8 == 0, "fm_router_backward: D must be a positive multiple of 8");
  FM_REQUIRE(ld_dl >= E && ld_x >= D && ld_x % 8 == 0 && (w == nullptr || (ld_w >= D && ld_w % 4 == 0)),
             "fm_router_backward: bad pitches");
  FM_REQUIRE(dx == nullptr || (ld_dx >= D && ld_dx % 8 == 0), "fm_router_backward: bad dx pitch");
  FM_REQUIRE(dw == nullptr || (ld_dw >= D), "fm_router_backward: bad dw pitch");
  if (dw != nullptr || db != nullptr)
    FM_REQUIRE(workspace != nullptr && workspace_bytes >= fm_router_workspace_bytes(T, D, E),
               "fm_router_backward: workspace of fm_router_workspace_bytes(T, D, E) bytes required");
  if (T == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  RouterBwdArgs a{dlogits, ld_dl, x, ld_x, T, D, w, ld_w, w_dtype == FM_DTYPE_BF16, E, dx, ld_dx,
                  static_cast<float*>(workspace), nullptr, 1, T};
  if (dx != nullptr) {
    const dim3 grid(unsigned((T + kRouterRows - 1) / kRouterRows));
    if (x_dtype == FM_DTYPE_BF16) hipLaunchKernelGGL((router_dx_kernel<uint16_t>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((router_dx_kernel<float>), grid, dim3(256), 0, s, a);
    if (int rc = check_launch("fm_router_backward")) return rc;
  }
  if (dw != nullptr || db != nullptr) {
    a.slices = router_slices(T, D, E);
    a.rows_per_slice = (T + a.slices - 1) / a.slices;
    a.part_db = db != nullptr ? a.part + a.slices * int64_t(E) * D : nullptr;
    const dim3 grid(unsigned((D + kDwCols - 1) / kDwCols), unsigned(a.slices), unsigned((E + 7) / 8));
    if (x_dtype == FM_DTYPE_BF16) hipLaunchKernelGGL((router_dw_kernel<uint16_t>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((router_dw_kernel<float>), grid, dim3(256), 0, s, a);
    if (int rc = check_launch("fm_router_backward")) return rc;
    const unsigned rblocks = unsigned((int64_t(E) * D + 63) / 64) + 1;
    hipLaunchKernelGGL(router_dw_reduce_kernel, dim3(rblocks), dim3(256), 0, s, a, dw, ld_dw,
                       int(dw_dtype == FM_DTYPE_BF16), db, int(db_dtype == FM_DTYPE_BF16));
    return check_launch("fm_router_backward");
  }
  return 0;
}

}  // extern "C"
