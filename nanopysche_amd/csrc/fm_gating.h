// Top-k gating of one group of tokens inside a wave (reference
// MoERouter._softmax_gating / _sigmoid_gating / R3 replay and the weight
// normalisation, model/moe.py:158-184, :249-265), shared by the gating kernel
// and the fused router forward.
//
// Lane layout: lane = g * EP + e for token slot g (64 / EP tokens per wave) and
// expert e < EP (EP = a power of two >= E); every reduction runs over the EP
// lanes of a slot with shuffles.
#pragma once

#include "fm_common.h"

namespace fm {

// Selection order of top-k: NaN above every number (as torch.topk orders
// it), then the larger value, then the lower expert index.
__device__ __forceinline__ bool beats(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ai < bi);
  return av > bv || (av == bv && ai < bi);
}

__device__ __forceinline__ int load_index(const void* p, int i64, int64_t i) {
  return i64 ? int(static_cast<const int64_t*>(p)[i]) : static_cast<const int32_t*>(p)[i];
}

__device__ __forceinline__ void store_index(void* p, int i64, int64_t i, int v) {
  if (i64) static_cast<int64_t*>(p)[i] = v;
  else static_cast<int32_t*>(p)[i] = v;
}

struct GateOut {
  int E, K;
  int sigmoid;           // sigmoid scores (else softmax over the K selected logits)
  int l2;                // divide the K weights by their l2 norm (+1e-8)
  const void* replay;    // [T, K] experts to replay (R3), or null
  int replay_i64;
  float* w;              // [T, K]
  void* idx;             // [T, K] int64 or int32
  int idx_i64;
  int need_p;            // softmax over all E needed (partials, replay or z-loss)
};

// Gating of token t (valid when tv) whose logit for expert e (lane's) is v
// (-inf for e >= E).  Writes w and idx for slots e < K; adds the lane's
// softmax probability to psum and logsumexp^2 to zsum (lane e == 0); returns
// the expert of slot e for lanes e < K (undefined elsewhere).
//   softmax:  top-k of the logits, w = softmax over the K selected logits
//   sigmoid:  top-k of sigmoid(logits), w = s / (sum s + 1e-8)
//   replay:   p = softmax(all logits), w_e = p_e / max(sum over the replayed
//             experts of p, 1e-8) on the replayed experts and 0 elsewhere
// Each of the K rounds is an arg-max over the experts not yet taken, so an
// expert never wins twice even when every remaining score is -inf.
template <int EP>
__device__ __forceinline__ int gate_group(const GateOut& a, int64_t t, bool tv, int g, int e, float v, float& psum,
                                          float& zsum) {
  const bool ev = e < a.E;
  float sc = a.sigmoid ? 1.f / (1.f + expf(-v)) : v;
  if (a.need_p) {
    float m = v;
#pragma unroll
    for (int off = EP / 2; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    float p = ev ? expf(v - m) : 0.f;
    float sm = p;
#pragma unroll
    for (int off = EP / 2; off > 0; off >>= 1) sm += __shfl_xor(sm, off);
    p /= sm;
    if (tv) psum += p;
    const float lse = m + logf(sm);
    if (tv && e == 0) zsum += lse * lse;
    if (a.replay) {
      const int r = (tv && e < a.K) ? load_index(a.replay, a.replay_i64, t * a.K + e) : -1;
      bool hit = false;
      for (int k = 0; k < a.K; ++k) hit |= __shfl(r, g * EP + k) == e;
      sc = (ev && hit) ? p : 0.f;
      float msum = sc;
#pragma unroll
      for (int off = EP / 2; off > 0; off >>= 1) msum += __shfl_xor(msum, off);
      sc /= fmaxf(msum, 1e-8f);
    }
  }
  bool taken = false;
  float top_first = 0.f, wsum = 0.f, my_w = 0.f;
  int my_i = 0;
  for (int k = 0; k < a.K; ++k) {
    const bool cand = ev && !taken;
    float bv = cand ? sc : -INFINITY;
    int bi = cand ? e : 0x7fffffff;
#pragma unroll
    for (int off = EP / 2; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off);
      const int oi = __shfl_xor(bi, off);
      if (beats(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (bi == e) taken = true;   // the winner leaves the race
    const float lg = __shfl(v, g * EP + (bi & (EP - 1)));
    if (k == 0) top_first = lg;
    const float wk = (a.sigmoid || a.replay) ? bv : expf(lg - top_first);
    wsum += wk;
    if (e == k) { my_w = wk; my_i = bi; }
  }
  float wn = a.replay ? my_w : (a.sigmoid ? my_w / (wsum + 1e-8f) : my_w / wsum);
  if (a.l2) {
    float sq = e < a.K ? wn * wn : 0.f;
#pragma unroll
    for (int off = EP / 2; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
    wn = wn / (sqrtf(sq) + 1e-8f);
  }
  if (tv && e < a.K) {
    a.w[t * a.K + e] = wn;
    store_index(a.idx, a.idx_i64, t * a.K + e, my_i);
  }
  return my_i;
}

}  // namespace fm
