// Router gate of the MoE layer (reference MoERouter.forward, model/moe.py:133-184):
//   fm_router_logits     logits[t][e] = sum_d x[t][d] * w[e][d] + bias[e] + score_bias[e], fp32
//                        (the reference's gate(x.float()) + score_bias, :151-154)
//   fm_expert_counts     counts[e] = number of the T*K slots routed to e (the f_i of the
//                        load-balancing loss, :267-281)
//   fm_gating_grad       dlogits from the gradient of the top-k weights (softmax over the K
//                        selected logits, :249-255, or normalised sigmoid, :257-265) plus the
//                        gradient of the load-balancing loss E * sum_i f_i P_i
//   fm_router_backward   dx = dlogits w, dw = dlogits^T x, db = sum_t dlogits (fp32; dw and
//                        db summed in a fixed order: dw as per-slice partials in a caller
//                        workspace, then the slices in order; db as one tree per expert)
//
// The gate is a skinny GEMM (E <= 256 outputs per token): x is read once at
// its size and the FMAs run on the VALU in fp32, as the reference computes it;
// HBM, not arithmetic, bounds it at the layer's shapes.
#include "fm_common.h"
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

// Stages w[e0 .. e0+EC)[c0 .. c0+kRouterCols) into LDS (zero past E or D).
// All of a thread's loads are issued before its LDS stores (a fixed trip
// count), so staging costs one memory latency, not one per element group.
template <int EC>
__device__ __forceinline__ void stage_gate(float (&wl)[EC][kRouterCols], const float* w, int64_t ld_w, int E,
                                           int64_t D, int e0, int64_t c0) {
  constexpr int kPer = EC * kRouterCols / 4 / 256;
  float4 v[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int i = threadIdx.x + 256 * u;
    const int e = i / (kRouterCols / 4), c = (i % (kRouterCols / 4)) * 4;
    v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e0 + e < E && c0 + c < D) v[u] = *reinterpret_cast<const float4*>(w + (e0 + e) * ld_w + c0 + c);
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
  const float* w;
  int64_t ld_w;
  const float* bias;
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
    stage_gate<EC>(wl, a.w, a.ld_w, a.E, a.D, e0, c0);
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
        if (a.bias) v += a.bias[eg];
        if (a.score_bias) v += a.score_bias[eg];
        a.logits[(r0 + r) * a.ld_l + eg] = v;
      }
    }
}

// Small gates (E <= 8, D <= 2048, D % 512 == 0): the whole gate sits in LDS (dynamic, 8 D
// floats, at most 64 KiB: two workgroups per CU), staged once, and each wave
// walks its 4 rows over D with the next 512-column chunk of x already in
// flight (no barrier inside the loop).
constexpr int kGateLdsFloats = 16 * 1024;

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
__device__ __forceinline__ void router_fma_chunk(float (&acc)[32], const float (&xv)[4][8], const float* wc,
                                                 int64_t D) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float4 w0 = *reinterpret_cast<const float4*>(wc + e * D);
    const float4 w1 = *reinterpret_cast<const float4*>(wc + e * D + 4);
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[r * 8 + e] = fmaf(xv[r][j], wv[j], acc[r * 8 + e]);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void router_logits_small_kernel(RouterArgs a) {
  extern __shared__ __attribute__((aligned(16))) float wl[];   // [8][D]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = int64_t(blockIdx.x) * kRouterRows + wave * 4;
  const int64_t D = a.D;
  const int nc = int(D / kRouterCols);   // D % 512 == 0 (launcher)
  // rows past T re-read the last row (their sums are not stored)
  const T* rows[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t row = r0 + r < a.T ? r0 + r : a.T - 1;
    rows[r] = static_cast<const T*>(a.x) + row * a.ld_x + lane * 8;
  }
  // bf16 rows of at most 2048 columns: all of this wave's x loads are issued
  // before the gate staging, so the two memory latencies overlap and the
  // chunk loop waits on none
  constexpr bool kWhole = sizeof(T) == 2;
  const bool whole = kWhole && nc <= 4;
  uint4 xr[4][4];
  if (whole) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (c < nc) xr[c][r] = *reinterpret_cast<const uint4*>(rows[r] + int64_t(c) * kRouterCols);
  }
  {
    // 8 gate rows of D <= 2048 floats over 256 threads: per row at most two
    // float4 per thread (expert x column loop, no index division), all loads
    // issued before the stores
    constexpr int kPerRow = kGateLdsFloats / 8 / 1024;
    float4 v[8][kPerRow];
    const int Di = int(D);
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int u = 0; u < kPerRow; ++u) {
        const int c = (int(threadIdx.x) + 256 * u) * 4;
        v[e][u] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c < Di && e < a.E) v[e][u] = *reinterpret_cast<const float4*>(a.w + e * a.ld_w + c);
      }
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
  const float sum = wave_reduce_scatter32(acc, lane);
  const int vi = lane >> 1, r = vi >> 3, e = vi & 7;
  if ((lane & 1) == 0 && e < a.E && r0 + r < a.T) {
    float v = sum;
    if (a.bias) v += a.bias[e];
    if (a.score_bias) v += a.score_bias[e];
    a.logits[(r0 + r) * a.ld_l + e] = v;
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
};

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
__global__ __launch_bounds__(256) void gating_grad_kernel(GatingGradArgs a) {
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
    if (a.dw) {
      // slots outside [0, E) carry no weight and no gradient
      int ik = -1;
      float lk = -INFINITY, dk = 0.f;
      if (lane < a.K) {
        const int64_t i = int64_t(t) * a.K + lane;
        ik = a.idx_i64 ? int(static_cast<const int64_t*>(a.idx)[i]) : static_cast<const int32_t*>(a.idx)[i];
        if (ik >= 0 && ik < a.E) {
          lk = a.logits[t * a.ld_l + ik];
          dk = a.dw[i];
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
  const float* w;        // [E, ld_w]
  int64_t ld_w;
  int E;
  void* dx;              // [T, ld_dx], x's dtype (null: skip)
  int64_t ld_dx;
  float* part;           // [slices][E][D] partial dw
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
      stage_gate<16>(wl, a.w, a.ld_w, a.E, a.D, e0, c0);
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

// Partial dw: grid (ceil(D / 512), slices, ceil(E / 8)); the slice's rows are
// split over the 4 waves (row t of the slice to wave t % 4), lane l owns
// columns 8 l .. of the chunk for 8 experts; the 4 waves' sums meet in LDS
// in a fixed order.
template <typename T>
__global__ __launch_bounds__(256) void router_dw_kernel(RouterBwdArgs a) {
  constexpr int EG = 8;
  __shared__ __attribute__((aligned(16))) float red[4][EG][kRouterCols];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t col = int64_t(blockIdx.x) * kRouterCols + lane * 8;
  const int64_t s = blockIdx.y;
  const int e0 = blockIdx.z * EG;
  const int64_t t_lo = s * a.rows_per_slice;
  const int64_t t_hi = t_lo + a.rows_per_slice < a.T ? t_lo + a.rows_per_slice : a.T;
  const T* x = static_cast<const T*>(a.x);
  float acc[EG][8];
#pragma unroll
  for (int e = 0; e < EG; ++e)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[e][j] = 0.f;
  if (col < a.D) {
    int64_t t = t_lo + wave;
    // four of the wave's rows per round: all their loads before any FMA (one
    // memory latency per four rows), the FMAs in row order as below
    for (; t + 12 < t_hi; t += 16) {
      float xv[4][8], dv[4][EG];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        load8f(x + (t + 4 * u) * a.ld_x + col, xv[u]);
#pragma unroll
        for (int e = 0; e < EG; ++e) dv[u][e] = e0 + e < a.E ? a.dl[(t + 4 * u) * a.ld_dl + e0 + e] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < EG; ++e)
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[e][j] = fmaf(dv[u][e], xv[u][j], acc[e][j]);
    }
    for (; t < t_hi; t += 4) {
      float xv[8];
      load8f(x + t * a.ld_x + col, xv);
#pragma unroll
      for (int e = 0; e < EG; ++e) {
        const float d = e0 + e < a.E ? a.dl[t * a.ld_dl + e0 + e] : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[e][j] = fmaf(d, xv[j], acc[e][j]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < EG; ++e)
#pragma unroll
    for (int j = 0; j < 8; ++j) red[wave][e][lane * 8 + j] = acc[e][j];
  __syncthreads();
  for (int i = threadIdx.x; i < EG * kRouterCols; i += 256) {
    const int e = i / kRouterCols, c = i % kRouterCols;
    const int64_t gc = int64_t(blockIdx.x) * kRouterCols + c;
    if (e0 + e < a.E && gc < a.D)
      a.part[(s * a.E + e0 + e) * a.D + gc] = ((red[0][e][c] + red[1][e][c]) + red[2][e][c]) + red[3][e][c];
  }
}

// dw[e][d] = sum over slices (in order) of the partials.
__global__ __launch_bounds__(256) void router_dw_reduce_kernel(RouterBwdArgs a, float* dw, int64_t ld_dw) {
  const int64_t n = int64_t(a.E) * a.D;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
    float v = 0.f;
#pragma unroll 8
    for (int64_t s = 0; s < a.slices; ++s) v += a.part[s * n + i];
    dw[(i / a.D) * ld_dw + i % a.D] = v;
  }
}

// db[e] = sum_t dl[t][e]: workgroup e, tokens strided over the threads, then
// a fixed-order tree in LDS.
__global__ __launch_bounds__(256) void router_db_kernel(const float* dl, int64_t ld_dl, int64_t T, float* db) {
  __shared__ float red[256];
  const int e = blockIdx.x;
  float v = 0.f;
  // unrolled so the loads of several rows are in flight at once; the adds
  // keep their order
#pragma unroll 8
  for (int64_t t = threadIdx.x; t < T; t += 256) v += dl[t * ld_dl + e];
  red[threadIdx.x] = v;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) db[e] = red[0];
}

// slices of the token range for the dw partials: at most 64, and at most
// 32 MiB of partials
inline int64_t router_slices(int64_t T, int64_t D, int E) {
  int64_t s = (32ll << 20) / (int64_t(E) * D * 4);
  s = s < 64 ? s : 64;
  s = s < 1 ? 1 : s;
  const int64_t per = (T + s - 1) / s;
  return per > 0 ? (T + per - 1) / per : 1;
}

}  // namespace fm

using namespace fm;

extern "C" {

int fm_router_logits(const void* x, int x_dtype, int64_t ld_x, int64_t T, int64_t D, const float* w,
                     int64_t ld_w, const float* bias, const float* score_bias, int E, float* logits,
                     int64_t ld_l, void* stream) {
  FM_REQUIRE(x && w && logits, "fm_router_logits: null pointer");
  FM_REQUIRE(x_dtype == FM_DTYPE_BF16 || x_dtype == FM_DTYPE_F32, "fm_router_logits: bad x dtype %d", x_dtype);
  FM_REQUIRE(E >= 1 && E <= 256, "fm_router_logits: E must be in [1, 256] (got %d)", E);
  FM_REQUIRE(D > 0 && D % 8 == 0, "fm_router_logits: D must be a positive multiple of 8 (got %lld)", (long long)D);
  FM_REQUIRE(ld_x >= D && ld_x % 8 == 0 && ld_w >= D && ld_w % 4 == 0 && ld_l >= E,
             "fm_router_logits: bad pitches");
  if (T == 0) return 0;
  const RouterArgs a{x, ld_x, T, D, w, ld_w, bias, score_bias, E, logits, ld_l};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned rb = unsigned((T + kRouterRows - 1) / kRouterRows);
  if (E <= 8 && 8 * D <= kGateLdsFloats && D % kRouterCols == 0) {
    const size_t lds = size_t(8 * D) * sizeof(float);
    if (x_dtype == FM_DTYPE_BF16) hipLaunchKernelGGL((router_logits_small_kernel<uint16_t>), dim3(rb), dim3(256), lds, s, a);
    else hipLaunchKernelGGL((router_logits_small_kernel<float>), dim3(rb), dim3(256), lds, s, a);
  } else if (E <= 8) {
    const dim3 grid(rb, 1);
    if (x_dtype == FM_DTYPE_BF16) hipLaunchKernelGGL((router_logits_kernel<uint16_t, 8>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((router_logits_kernel<float, 8>), grid, dim3(256), 0, s, a);
  } else {
    const dim3 grid(rb, unsigned((E + 15) / 16));
    if (x_dtype == FM_DTYPE_BF16) hipLaunchKernelGGL((router_logits_kernel<uint16_t, 16>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((router_logits_kernel<float, 16>), grid, dim3(256), 0, s, a);
  }
  return check_launch("fm_router_logits");
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
  FM_REQUIRE(logits && indices && dlogits, "fm_gating_grad: null pointer");
  FM_REQUIRE(E >= 1 && E <= 64 * kGateMaxPerLane, "fm_gating_grad: E must be in [1, %d] (got %d)",
             64 * kGateMaxPerLane, E);
  FM_REQUIRE(K >= 1 && K <= E && K <= 64, "fm_gating_grad: K must be in [1, min(E, 64)] (got %d)", K);
  FM_REQUIRE(gating == FM_GATING_SOFTMAX || gating == FM_GATING_SIGMOID, "fm_gating_grad: bad gating");
  FM_REQUIRE((flags & ~FM_GATING_L2_NORMALIZE) == 0, "fm_gating_grad: unknown flags 0x%x", flags);
  FM_REQUIRE(daux == nullptr || counts != nullptr, "fm_gating_grad: the aux-loss gradient needs counts");
  FM_REQUIRE(ld_l >= E && ld_d >= E, "fm_gating_grad: pitch < E");
  if (T == 0) return 0;
  const GatingGradArgs a{logits, T, ld_l, E, K, (gating == FM_GATING_SIGMOID && !replay) ? 1 : 0,
                         (flags & FM_GATING_L2_NORMALIZE) ? 1 : 0, indices, indices_i64, dweights, daux,
                         counts, z_loss_multiplier, dlogits, ld_d};
  const int64_t blocks = (T + 3) / 4 < 4096 ? (T + 3) / 4 : 4096;
  hipLaunchKernelGGL(gating_grad_kernel, dim3(unsigned(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("fm_gating_grad");
}

int64_t fm_router_workspace_bytes(int64_t T, int64_t D, int E) {
  if (T <= 0 || D <= 0 || E <= 0) return 0;
  return router_slices(T, D, E) * int64_t(E) * D * int64_t(sizeof(float));
}

int fm_router_backward(const float* dlogits, int64_t ld_dl, const void* x, int x_dtype, int64_t ld_x, int64_t T,
                       int64_t D, const float* w, int64_t ld_w, int E, void* dx, int64_t ld_dx, float* dw,
                       int64_t ld_dw, float* db, void* workspace, int64_t workspace_bytes, void* stream) {
  FM_REQUIRE(dlogits && x && (w || dx == nullptr), "fm_router_backward: null pointer");
  FM_REQUIRE(x_dtype == FM_DTYPE_BF16 || x_dtype == FM_DTYPE_F32, "fm_router_backward: bad x dtype %d", x_dtype);
  FM_REQUIRE(E >= 1 && E <= 256, "fm_router_backward: E must be in [1, 256] (got %d)", E);
  FM_REQUIRE(D > 0 && D % 8 == 0, "fm_router_backward: D must be a positive multiple of 8");
  FM_REQUIRE(ld_dl >= E && ld_x >= D && ld_x % 8 == 0 && (w == nullptr || (ld_w >= D && ld_w % 4 == 0)),
             "fm_router_backward: bad pitches");
  FM_REQUIRE(dx == nullptr || (ld_dx >= D && ld_dx % 8 == 0), "fm_router_backward: bad dx pitch");
  FM_REQUIRE(dw == nullptr || (ld_dw >= D), "fm_router_backward: bad dw pitch");
  if (dw != nullptr)
    FM_REQUIRE(workspace != nullptr && workspace_bytes >= fm_router_workspace_bytes(T, D, E),
               "fm_router_backward: workspace of fm_router_workspace_bytes(T, D, E) bytes required");
  if (T == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  RouterBwdArgs a{dlogits, ld_dl, x, ld_x, T, D, w, ld_w, E, dx, ld_dx, static_cast<float*>(workspace), 1, T};
  if (dx != nullptr) {
    const dim3 grid(unsigned((T + kRouterRows - 1) / kRouterRows));
    if (x_dtype == FM_DTYPE_BF16) hipLaunchKernelGGL((router_dx_kernel<uint16_t>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((router_dx_kernel<float>), grid, dim3(256), 0, s, a);
    if (int rc = check_launch("fm_router_backward")) return rc;
  }
  if (dw != nullptr) {
    a.slices = router_slices(T, D, E);
    a.rows_per_slice = (T + a.slices - 1) / a.slices;
    const dim3 grid(unsigned((D + kRouterCols - 1) / kRouterCols), unsigned(a.slices), unsigned((E + 7) / 8));
    if (x_dtype == FM_DTYPE_BF16) hipLaunchKernelGGL((router_dw_kernel<uint16_t>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((router_dw_kernel<float>), grid, dim3(256), 0, s, a);
    if (int rc = check_launch("fm_router_backward")) return rc;
    const int64_t n = int64_t(E) * D;
    const unsigned rblocks = unsigned((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024);
    hipLaunchKernelGGL(router_dw_reduce_kernel, dim3(rblocks), dim3(256), 0, s, a, dw, ld_dw);
    if (int rc = check_launch("fm_router_backward")) return rc;
  }
  if (db != nullptr) {
    hipLaunchKernelGGL(router_db_kernel, dim3(unsigned(E)), dim3(256), 0, s, dlogits, ld_dl, T, db);
    return check_launch("fm_router_backward");
  }
  return 0;
}

}  // extern "C"
