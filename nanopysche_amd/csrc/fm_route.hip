// Token routing for the expert block:
//   fm_topk_gating      -- softmax / sigmoid top-k over E experts, one wave64 per
//                          token, plus deterministic per-wave sums of the full
//                          softmax for the load-balancing loss
//   fm_aux_loss         -- E * sum_i f_i P_i from the counts and those sums
//   fm_route_sort       -- stable counting sort of the T*K (token, slot)
//                          assignments by expert: ballot-counted histograms per
//                          1024 assignments, per-expert wave scans,
//                          wave-ballot ranks; padded group offsets (multiples of
//                          128), row maps, and the m-tile -> expert table
//   fm_permute          -- gather x rows into the padded expert-contiguous
//                          buffer, optionally scaled by the router weight, fused
//                          with bf16 / e4m3 row and transposed outputs
//   fm_unpermute        -- out[t] = sum_k w[t,k] * y[row(t,k)], fp32 sum, one
//                          rounding
//   fm_router_weight_grad -- dw[t,k] = <dout[t], y[row(t,k)]>
//   fm_capacity_select  -- capacity dropping: ranks from the sort's rows, keep
//                          flags, then a block-count compaction of the kept tokens
//   fm_gather_rows      -- row gather with zero rows for index -1 (the kept
//                          tokens' selection and the scatter back)
#include <mutex>
#include <type_traits>

#include "fm_gating.h"
#include "fm_weight_tile.h"
#include "../../include/fm_hip.h"

namespace fm {

// ---------------------------------------------------------------- top-k ----
struct TopkArgs {
  const float* logits;   // [T, E] row pitch ld
  int64_t T, ld;
  int E, K;
  int sigmoid;
  int l2;                // normalise the K weights by their l2 norm (+1e-8)
  const void* replay;    // [T, K] experts to replay (R3), or null
  int replay_i64;
  float* w;              // [T, K]
  void* idx;             // [T, K] int64 or int32
  int idx_i64;
  float* prob_partial;   // [n_waves, E] or null: per-wave sums of softmax(logits)
  float* z_partial;      // [n_waves] or null: per-wave sums of logsumexp(logits)^2
};

constexpr int kTopkMaxPerLane = 4;  // E <= 256

// One token per wave; lane l holds experts l + 64 j.  Each of the K rounds is
// a wave arg-max over the experts not yet taken (a per-lane taken mask, so an
// expert never wins twice even when every remaining score is -inf).
//   softmax:  top-k of the logits, w = softmax over the K selected logits
//   sigmoid:  top-k of sigmoid(logits), w = s / (sum s + 1e-8)
//   replay:   p = softmax(all logits), w_e = p_e / max(sum over the replayed
//             experts of p, 1e-8) on the replayed experts and 0 elsewhere;
//             the K largest w in order (the reference's R3 gating)
// then optionally w / (||w||_2 + 1e-8).
__global__ __launch_bounds__(256) void topk_kernel(TopkArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t n_waves = int64_t(gridDim.x) * 4;
  const bool need_p = a.prob_partial || a.replay || a.z_partial;
  float psum[kTopkMaxPerLane];
#pragma unroll
  for (int j = 0; j < kTopkMaxPerLane; ++j) psum[j] = 0.f;
  float zsum = 0.f;
  for (int64_t t = wave; t < a.T; t += n_waves) {
    float v[kTopkMaxPerLane];   // logits of experts lane + 64*j
    float sc[kTopkMaxPerLane];  // selection scores
#pragma unroll
    for (int j = 0; j < kTopkMaxPerLane; ++j) {
      const int e = lane + 64 * j;
      v[j] = e < a.E ? a.logits[t * a.ld + e] : -INFINITY;
      sc[j] = a.sigmoid ? 1.f / (1.f + expf(-v[j])) : v[j];
    }
    if (need_p) {
      float m = -INFINITY;
#pragma unroll
      for (int j = 0; j < kTopkMaxPerLane; ++j) m = fmaxf(m, v[j]);
      for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
      float ex[kTopkMaxPerLane], s = 0.f;
#pragma unroll
      for (int j = 0; j < kTopkMaxPerLane; ++j) {
        ex[j] = (lane + 64 * j) < a.E ? expf(v[j] - m) : 0.f;
        s += ex[j];
      }
      for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
#pragma unroll
      for (int j = 0; j < kTopkMaxPerLane; ++j) {
        ex[j] /= s;
        psum[j] += ex[j];
      }
      const float lse = m + logf(s);
      zsum += lse * lse;
      if (a.replay) {
        // masked, renormalised probabilities become the selection scores
        const int r = lane < a.K ? load_index(a.replay, a.replay_i64, t * a.K + lane) : -1;
        float msum = 0.f;
#pragma unroll
        for (int j = 0; j < kTopkMaxPerLane; ++j) {
          bool hit = false;
          for (int k = 0; k < a.K; ++k) hit |= __shfl(r, k) == lane + 64 * j;
          sc[j] = hit ? ex[j] : 0.f;
          msum += sc[j];
        }
        for (int off = 32; off > 0; off >>= 1) msum += __shfl_xor(msum, off);
        msum = fmaxf(msum, 1e-8f);
#pragma unroll
        for (int j = 0; j < kTopkMaxPerLane; ++j) sc[j] /= msum;
      }
    }
    uint32_t taken = 0;
    float top_first = 0.f, wsum = 0.f, my_w = 0.f;
    int my_i = 0;
    for (int k = 0; k < a.K; ++k) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < kTopkMaxPerLane; ++j) {
        const int e = lane + 64 * j;
        if (e < a.E && !((taken >> j) & 1u) && beats(sc[j], e, bv, bi)) { bv = sc[j]; bi = e; }
      }
      for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (beats(ov, oi, bv, bi)) { bv = ov; bi = oi; }
      }
      const int jw = bi >> 6;   // bi < E: K <= E candidates exist in every round
      if ((bi & 63) == lane) taken |= 1u << jw;
      float vj = v[0];
#pragma unroll
      for (int j = 1; j < kTopkMaxPerLane; ++j) vj = jw == j ? v[j] : vj;
      const float lg = __shfl(vj, bi & 63);
      if (k == 0) top_first = lg;
      // sigmoid and replay weights are the scores; softmax: exp(l - l_max)
      const float wk = (a.sigmoid || a.replay) ? bv : expf(lg - top_first);
      wsum += wk;
      if (lane == k) { my_w = wk; my_i = bi; }
    }
    float wn = a.replay ? my_w : (a.sigmoid ? my_w / (wsum + 1e-8f) : my_w / wsum);
    if (a.l2) {
      float sq = lane < a.K ? wn * wn : 0.f;
      for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
      wn = wn / (sqrtf(sq) + 1e-8f);
    }
    if (lane < a.K) {
      a.w[t * a.K + lane] = wn;
      store_index(a.idx, a.idx_i64, t * a.K + lane, my_i);
    }
  }
  if (a.prob_partial) {
#pragma unroll
    for (int j = 0; j < kTopkMaxPerLane; ++j) {
      const int e = lane + 64 * j;
      if (e < a.E) a.prob_partial[wave * a.E + e] = psum[j];
    }
  }
  if (a.z_partial && lane == 0) a.z_partial[wave] = zsum;
}

// E <= 16: a wave takes 64 / EP tokens at once (EP = E rounded up to a power
// of two; lane = token slot * EP + expert), so the reductions run over EP
// lanes (log2 EP steps) for NT tokens together instead of over 64 lanes for
// one token.  Same selection rule, weights (sum over k in k order), replay,
// l2 normalisation and per-wave partials as topk_kernel.
template <int EP>
__global__ __launch_bounds__(256) void topk_small_kernel(TopkArgs a) {
  constexpr int NT = 64 / EP;
  const int lane = threadIdx.x & 63, g = lane / EP, e = lane % EP;
  const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t n_waves = int64_t(gridDim.x) * 4;
  const GateOut go{a.E, a.K, a.sigmoid, a.l2, a.replay, a.replay_i64, a.w, a.idx, a.idx_i64,
                   (a.prob_partial || a.replay || a.z_partial) ? 1 : 0};
  float psum = 0.f, zsum = 0.f;
  for (int64_t tg = wave; tg * NT < a.T; tg += n_waves) {
    const int64_t t = tg * NT + g;
    const bool tv = t < a.T;
    const float v = (tv && e < a.E) ? a.logits[t * a.ld + e] : -INFINITY;
    gate_group<EP>(go, t, tv, g, e, v, psum, zsum);
  }
  if (a.prob_partial) {
#pragma unroll
    for (int off = EP; off < 64; off <<= 1) psum += __shfl_xor(psum, off);
    if (lane < a.E) a.prob_partial[wave * a.E + lane] = psum;
  }
  if (a.z_partial) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) zsum += __shfl_xor(zsum, off);
    if (lane == 0) a.z_partial[wave] = zsum;
  }
}

// one block of 512 threads: wave w sums experts w, w + 8, ... -- each lane a
// strided run of the per-wave partials, then a fixed shuffle tree -- so no
// workgroup barrier sits inside the per-expert sums; thread 0 then adds
// f_e * P_e in expert order.  loss = E * sum_e f_e P_e, P_e = sum / T, plus
// z_mult * (sum of the per-wave logsumexp^2 partials) / T when z_partial is
// given (the z-loss of model/moe.py:176-178).
__global__ __launch_bounds__(512) void aux_loss_kernel(const float* prob_partial, int64_t n_waves,
                                                       const int32_t* counts, int E, int64_t T,
                                                       const float* z_partial, float z_mult, float* loss) {
  __shared__ float term[1024];   // E <= 1024 (launcher)
  __shared__ float zterm;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int e = wave; e < E; e += 8) {
    float p = 0.f;
    for (int64_t w = lane; w < n_waves; w += 64) p += prob_partial[w * E + e];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) p += __shfl_xor(p, off);
    if (lane == 0) term[e] = (float(counts[e]) / float(T)) * (p / float(T));
  }
  if (wave == 7) {
    float z = 0.f;
    if (z_partial)
      for (int64_t w = lane; w < n_waves; w += 64) z += z_partial[w];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) z += __shfl_xor(z, off);
    if (lane == 0) zterm = z / float(T);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float acc = 0.f;
    for (int e = 0; e < E; ++e) acc += term[e];
    float l = float(E) * acc;
    if (z_partial) l = l + z_mult * zterm;
    loss[0] = l;
  }
}

// ----------------------------------------------------------------- sort ----
constexpr int kSortBlock = 1024;     // assignments per workgroup (256 per wave)
constexpr int kSortMaxExperts = 1024;

template <typename I>
__device__ __forceinline__ int load_expert(const I* idx, int64_t a, int E) {
  const int64_t e = int64_t(idx[a]);
  return (e >= 0 && e < E) ? int(e) : -1;
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Lanes of the wave holding the same expert as this lane (one ballot per
// expert-id bit); e < 0 marks lanes with no assignment.
__device__ __forceinline__ uint64_t expert_peers(int e, int nbits) {
  uint64_t peers = __ballot(e >= 0);
#pragma unroll 1
  for (int b = 0; b < nbits; ++b) {
    const uint64_t ones = __ballot(e >= 0 && ((e >> b) & 1));
    peers &= ((e >> b) & 1) ? ones : ~ones;
  }
  return e >= 0 ? peers : 0ull;
}

__device__ __forceinline__ int expert_bits(int E) {
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  return nbits;
}

// block_hist[e][b] = assignments of block b routed to expert e.  Each wave
// counts 64 assignments at a time; the lowest lane of every group of equal
// experts adds the group's size (one LDS atomic per distinct expert).
template <typename I>
__global__ __launch_bounds__(256) void sort_hist_kernel(const I* idx, int64_t A, int E,
                                                        int32_t* block_hist, int64_t n_blocks, WeightSide side) {
  if (int64_t(blockIdx.x) >= n_blocks) {   // workgroups past the sort's run expert-weight blocks
    weight_side_block(side, int64_t(blockIdx.x) - n_blocks);
    return;
  }
  __shared__ int32_t hist[kSortMaxExperts];
  for (int e = threadIdx.x; e < E; e += 256) hist[e] = 0;
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nbits = expert_bits(E);
  const int64_t q0 = int64_t(blockIdx.x) * kSortBlock + int64_t(wave) * (kSortBlock / 4);
  for (int i0 = 0; i0 < kSortBlock / 4; i0 += 64) {
    const int64_t a = q0 + i0 + lane;
    const int e = a < A ? load_expert(idx, a, E) : -1;
    const uint64_t peers = expert_peers(e, nbits);
    if (e >= 0 && (peers & lanemask_lt()) == 0) atomicAdd(&hist[e], __popcll(peers));
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 256) block_hist[int64_t(e) * n_blocks + blockIdx.x] = hist[e];
}

// One block of 1024 threads (16 waves).  Wave w scans experts w, w + 16, ...:
// block_hist[e][*] becomes its exclusive prefix over blocks (64 blocks per
// pass, wave prefix sums).  Then counts, padded offsets, the m-tile -> expert
// map and the per-expert FP8/BF16 flag are written; assign_of_row is reset to
// -1.
__global__ __launch_bounds__(1024) void sort_scan_kernel(int32_t* block_hist, int64_t n_blocks,
                                                         int E, int32_t* counts, int32_t* offsets,
                                                         int32_t* tile_expert, int64_t n_tiles_max,
                                                         int32_t* assign_of_row, int64_t rows_max,
                                                         int32_t* use_fp8, int64_t threshold) {
  __shared__ int32_t padded[kSortMaxExperts];
  __shared__ int32_t scan[kSortMaxExperts + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = wave; e < E; e += 16) {
    int32_t* h = block_hist + int64_t(e) * n_blocks;
    int32_t run = 0;
    for (int64_t b0 = 0; b0 < n_blocks; b0 += 64) {
      const int64_t b = b0 + lane;
      const int32_t v = b < n_blocks ? h[b] : 0;
      int32_t incl = v;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int32_t o = __shfl_up(incl, off);
        if (lane >= off) incl += o;
      }
      if (b < n_blocks) h[b] = run + incl - v;
      run += __shfl(incl, 63);
    }
    if (lane == 0) {
      counts[e] = run;
      padded[e] = (run + 127) / 128 * 128;
      if (use_fp8) use_fp8[e] = int64_t(run) >= threshold ? 1 : 0;
    }
  }
  __syncthreads();
  if (tid == 0) {
    int32_t s = 0;
    for (int e = 0; e < E; ++e) { scan[e] = s; s += padded[e]; }
    scan[E] = s;
  }
  __syncthreads();
  for (int e = tid; e <= E; e += 1024) offsets[e] = scan[e];
  const int64_t used_tiles = scan[E] / 128;
  for (int64_t m = tid; m < n_tiles_max; m += 1024) {
    int32_t ex = -1;
    if (m < used_tiles) {
      // binary search: last e with scan[e] <= 128*m
      int lo = 0, hi = E - 1;
      const int32_t r = int32_t(m * 128);
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (scan[mid] <= r) lo = mid; else hi = mid - 1;
      }
      ex = lo;
    }
    tile_expert[m] = ex;
  }
  for (int64_t r = tid; r < rows_max; r += 1024) assign_of_row[r] = -1;
}

// Each wave owns a contiguous quarter (256 assignments) of the block and
// walks it 64 at a time; peers with the same expert are found with one ballot
// per expert-id bit, so ranks follow assignment order (stable).
template <typename I>
__global__ __launch_bounds__(256) void sort_scatter_kernel(const I* idx, int64_t A, int E,
                                                           const int32_t* block_prefix, int64_t n_blocks,
                                                           const int32_t* offsets,
                                                           int32_t* row_of,
                                                           int32_t* assign_of_row) {
  __shared__ int32_t base[4][kSortMaxExperts];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nbits = expert_bits(E);
  for (int i = threadIdx.x; i < 4 * E; i += 256) base[i / E][i % E] = 0;
  __syncthreads();
  const int64_t q0 = int64_t(blockIdx.x) * kSortBlock + int64_t(wave) * (kSortBlock / 4);
  for (int i0 = 0; i0 < kSortBlock / 4; i0 += 64) {
    const int64_t a = q0 + i0 + lane;
    const int e = a < A ? load_expert(idx, a, E) : -1;
    const uint64_t peers = expert_peers(e, nbits);
    if (e >= 0 && (peers & lanemask_lt()) == 0) atomicAdd(&base[wave][e], __popcll(peers));
  }
  __syncthreads();
  // exclusive prefix over the 4 waves, plus the block prefix and group offset
  for (int e = threadIdx.x; e < E; e += 256) {
    int32_t run = offsets[e] + block_prefix[int64_t(e) * n_blocks + blockIdx.x];
    for (int w = 0; w < 4; ++w) {
      const int32_t c = base[w][e];
      base[w][e] = run;
      run += c;
    }
  }
  __syncthreads();
  for (int i0 = 0; i0 < kSortBlock / 4; i0 += 64) {
    const int64_t a = q0 + i0 + lane;
    const int e = a < A ? load_expert(idx, a, E) : -1;
    const uint64_t peers = expert_peers(e, nbits);
    int32_t my_base = 0;
    if (e >= 0) my_base = base[wave][e];
    __builtin_amdgcn_wave_barrier();
    if (e >= 0) {
      const int32_t row = my_base + __popcll(peers & lanemask_lt());
      row_of[a] = row;
      assign_of_row[row] = int32_t(a);
      // lowest lane of the peer group advances the counter
      if ((peers & lanemask_lt()) == 0) base[wave][e] = my_base + __popcll(peers);
    } else if (a < A) {
      row_of[a] = -1;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// sort_scan_kernel and sort_scatter_kernel as one launch for at most
// kFusedBlocks blocks and kFusedExperts experts: each workgroup re-derives
// what the scan would hand it from the block table -- the expert totals,
// its own block prefix, the padded group starts -- so no workgroup waits on
// another.  Workgroup 0 writes counts, offsets, the m-tile table and the
// FP8 flags; the -1 of assign_of_row goes only to pad rows (after each
// group's last assignment, and past the last group), which the scatter
// never writes, split over the workgroups.  Same outputs as the two kernels.
constexpr int64_t kFusedBlocks = 64;
constexpr int kFusedExperts = 256;

template <typename I>
__global__ __launch_bounds__(256) void sort_scan_scatter_kernel(const I* idx, int64_t A, int E,
                                                                const int32_t* block_hist, int64_t n_blocks,
                                                                int32_t* counts, int32_t* offsets,
                                                                int32_t* tile_expert, int64_t n_tiles_max,
                                                                int32_t* row_of, int32_t* assign_of_row,
                                                                int64_t rows_max, int32_t* use_fp8,
                                                                int64_t threshold, WeightSide side) {
  if (int64_t(blockIdx.x) >= n_blocks) {   // workgroups past the sort's run expert-weight blocks
    weight_side_block(side, int64_t(blockIdx.x) - n_blocks);
    return;
  }
  __shared__ int32_t base[4][kFusedExperts];   // per-wave counts, then per-wave next rows
  __shared__ int32_t start[kFusedExperts + 1];  // padded group starts; start[E] = rows used
  __shared__ int32_t wtot[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nbits = expert_bits(E);
  for (int i = tid; i < 4 * kFusedExperts; i += 256) (&base[0][0])[i] = 0;
  // thread e: expert e's total and this block's prefix from the block table
  int32_t tot = 0, pre = 0;
  if (tid < E) {
    const int32_t* h = block_hist + int64_t(tid) * n_blocks;
    for (int64_t b0 = 0; b0 < n_blocks; b0 += 16) {
      int32_t v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = b0 + u < n_blocks ? h[b0 + u] : 0;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        tot += v[u];
        if (b0 + u < int64_t(blockIdx.x)) pre += v[u];
      }
    }
  }
  __syncthreads();
  const int64_t q0 = int64_t(blockIdx.x) * kSortBlock + int64_t(wave) * (kSortBlock / 4);
  for (int i0 = 0; i0 < kSortBlock / 4; i0 += 64) {
    const int64_t a = q0 + i0 + lane;
    const int e = a < A ? load_expert(idx, a, E) : -1;
    const uint64_t peers = expert_peers(e, nbits);
    if (e >= 0 && (peers & lanemask_lt()) == 0) atomicAdd(&base[wave][e], __popcll(peers));
  }
  // group starts: exclusive scan of the padded totals over the experts
  const int32_t pad = tid < E ? (tot + 127) / 128 * 128 : 0;
  int32_t incl = pad;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int32_t o = __shfl_up(incl, off);
    if (lane >= off) incl += o;
  }
  if (lane == 63) wtot[wave] = incl;
  __syncthreads();
  int32_t before = 0;
  for (int w = 0; w < wave; ++w) before += wtot[w];
  const int32_t st = before + incl - pad;
  if (tid < E) start[tid] = st;
  if (tid == 0) start[E] = wtot[0] + wtot[1] + wtot[2] + wtot[3];
  if (tid < E) {   // this wave-quarter's first rows: group start + block prefix + earlier quarters
    int32_t run = st + pre;
    for (int w = 0; w < 4; ++w) {
      const int32_t c = base[w][tid];
      base[w][tid] = run;
      run += c;
    }
    if (blockIdx.x == 0) {
      counts[tid] = tot;
      if (use_fp8) use_fp8[tid] = int64_t(tot) >= threshold ? 1 : 0;
    }
  }
  __syncthreads();
  const int32_t used = start[E];
  if (blockIdx.x == 0) {
    for (int e = tid; e <= E; e += 256) offsets[e] = start[e];
    for (int64_t m = tid; m < n_tiles_max; m += 256) {
      int32_t ex = -1;
      if (m * 128 < used) {   // last e with start[e] <= 128 m
        int lo = 0, hi = E - 1;
        const int32_t r = int32_t(m * 128);
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (start[mid] <= r) lo = mid; else hi = mid - 1;
        }
        ex = lo;
      }
      tile_expert[m] = ex;
    }
  }
  // pad rows: expert e's (fewer than 128) go to workgroup e % n_blocks, the
  // rows past the last group are strided over all workgroups
  if (tid < E && tid % n_blocks == int64_t(blockIdx.x)) {
    for (int32_t r = st + tot; r < start[tid + 1]; ++r) assign_of_row[r] = -1;
  }
  for (int64_t r = used + int64_t(blockIdx.x) * 256 + tid; r < rows_max; r += n_blocks * 256) assign_of_row[r] = -1;
  for (int i0 = 0; i0 < kSortBlock / 4; i0 += 64) {
    const int64_t a = q0 + i0 + lane;
    const int e = a < A ? load_expert(idx, a, E) : -1;
    const uint64_t peers = expert_peers(e, nbits);
    int32_t my_base = 0;
    if (e >= 0) my_base = base[wave][e];
    __builtin_amdgcn_wave_barrier();
    if (e >= 0) {
      const int32_t row = my_base + __popcll(peers & lanemask_lt());
      row_of[a] = row;
      assign_of_row[row] = int32_t(a);
      if ((peers & lanemask_lt()) == 0) base[wave][e] = my_base + __popcll(peers);
    } else if (a < A) {
      row_of[a] = -1;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// -------------------------------------------------------- tile masks ----
// Per-precision tile lists for the fp8_gemm_threshold split: tile t keeps
// its expert in tiles_fp8 when that expert takes the FP8 GEMMs, in
// tiles_bf16 otherwise, and -1 in the other list (and in both past the last
// group), so each producer writes only the rows its own GEMMs read.
__global__ __launch_bounds__(256) void tile_masks_kernel(const int32_t* __restrict__ tile_expert, int64_t n,
                                                         const int32_t* __restrict__ use_fp8,
                                                         int32_t* __restrict__ tiles_fp8,
                                                         int32_t* __restrict__ tiles_bf16) {
  for (int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x; t < n; t += int64_t(gridDim.x) * 256) {
    const int32_t e = tile_expert[t];
    const bool f = e >= 0 && use_fp8[e] != 0;
    tiles_fp8[t] = f ? e : -1;
    tiles_bf16[t] = e >= 0 && !f ? e : -1;
  }
}

// -------------------------------------------------------------- permute ----
// Row r of the padded buffer is x[assign_of_row[r] / K] (times the router
// weight of that assignment when WEIGHTED), zeros for pad rows.  Branch-free:
// a pad row reads assignment 0 and is zeroed by a select (the launcher uses
// ZeroSrc when there are no assignments).
template <bool WEIGHTED>
struct GatherSrc {
  static constexpr int kOut = 1;
  const uint16_t* x;  // bf16 [T, D]
  int64_t ld;
  const int32_t* assign_of_row;
  int K;
  const float* w;     // [T*K] (WEIGHTED)
  struct Raw {
    uint4 pk;
    float s;
    bool ok;
  };
  __device__ __forceinline__ Raw fetch(int64_t row, int64_t col) const {
    const int32_t a = assign_of_row[row];
    const int32_t ac = a >= 0 ? a : 0;
    Raw r;
    r.ok = a >= 0;
    r.pk = *reinterpret_cast<const uint4*>(x + int64_t(ac / K) * ld + col);
    r.s = WEIGHTED ? w[ac] : 1.f;
    return r;
  }
  __device__ __forceinline__ void compute(const Raw& r, float v[][8]) const {
    float f[8];
    unpack8_bf16(r.pk, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[0][i] = r.ok ? (WEIGHTED ? r.s * f[i] : f[i]) : 0.f;
  }
};

// All pad rows (no assignments at all).
struct ZeroSrc {
  static constexpr int kOut = 1;
  struct Raw {};
  __device__ __forceinline__ Raw fetch(int64_t, int64_t) const { return Raw{}; }
  __device__ __forceinline__ void compute(const Raw&, float v[][8]) const {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[0][i] = 0.f;
  }
};

// ------------------------------------------------------------ unpermute ----
// grid-stride over (token, 8-column chunk); K rows summed in slot order
// with separately rounded multiply and add (contraction into FMA is switched
// off for this kernel), one rounding to the output dtype at the end.
// KC > 0 (K == KC): a thread loads the token's KC row indices and weights,
// then issues every slot's row load before the first sum, instead of one
// index-then-row round trip per slot (at top-8 with most slots outside the
// local experts that chain was 8 dependent loads per token); the sums keep
// the slot order.  KC == 0: any K, one slot at a time.
template <int KC, bool VEC = false>   // VEC: row_of (and w) 16-byte aligned, KC in {4, 8}
__global__ __launch_bounds__(256) void unpermute_kernel(const uint16_t* __restrict__ y, int64_t ld_y,
                                                        const int32_t* __restrict__ row_of,
                                                        const float* __restrict__ w, int64_t T, int K,
                                                        int64_t D, void* __restrict__ out, int out_f32,
                                                        int64_t ld_out, const uint16_t* __restrict__ addend,
                                                        int64_t ld_add) {
#pragma clang fp contract(off)
  const int64_t chunks = D / 8;
  const int64_t n = T * chunks;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
    const int64_t t = i / chunks, c = (i % chunks) * 8;
    float acc[8];
    if (addend) {   // the sum starts from the addend's row (bf16)
      const uint4 pk = *reinterpret_cast<const uint4*>(addend + t * ld_add + c);
      const uint32_t q[4] = {pk.x, pk.y, pk.z, pk.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = u2f(q[j] << 16);
        acc[2 * j + 1] = u2f(q[j] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    }
    auto add_row = [&](uint4 pk, float s) {
      const uint32_t q[4] = {pk.x, pk.y, pk.z, pk.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = acc[2 * j] + s * u2f(q[j] << 16);
        acc[2 * j + 1] = acc[2 * j + 1] + s * u2f(q[j] & 0xffff0000u);
      }
    };
    if constexpr (KC > 0) {
      int32_t r[KC];
      float sw[KC];
      uint4 pk[KC];
      if constexpr (VEC) {   // a token's KC slots in 16-byte loads (KC = 8: sixteen 4-byte loads -> four)
        constexpr int V = 4;
#pragma unroll
        for (int k = 0; k < KC; k += V) {
          const int4 a = *reinterpret_cast<const int4*>(row_of + t * KC + k);
          r[k] = a.x; r[k + 1] = a.y; r[k + 2] = a.z; r[k + 3] = a.w;
          if (w) {
            const float4 b = *reinterpret_cast<const float4*>(w + t * KC + k);
            sw[k] = b.x; sw[k + 1] = b.y; sw[k + 2] = b.z; sw[k + 3] = b.w;
          } else {
#pragma unroll
            for (int j = 0; j < V; ++j) sw[k + j] = 1.f;
          }
        }
      } else {
#pragma unroll
        for (int k = 0; k < KC; ++k) {
          r[k] = row_of[t * KC + k];
          sw[k] = w ? w[t * KC + k] : 1.f;
        }
      }
#pragma unroll
      for (int k = 0; k < KC; ++k)
        pk[k] = r[k] >= 0 ? *reinterpret_cast<const uint4*>(y + int64_t(r[k]) * ld_y + c) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int k = 0; k < KC; ++k)
        if (r[k] >= 0) add_row(pk[k], sw[k]);
    } else {
      for (int k = 0; k < K; ++k) {
        const int32_t r = row_of[t * K + k];
        if (r < 0) continue;
        add_row(*reinterpret_cast<const uint4*>(y + int64_t(r) * ld_y + c), w ? w[t * K + k] : 1.f);
      }
    }
    if (out_f32) {
      float* o = static_cast<float*>(out) + t * ld_out + c;
      *reinterpret_cast<float4*>(o) = make_float4(acc[0], acc[1], acc[2], acc[3]);
      *reinterpret_cast<float4*>(o + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
    } else {
      uint4 pk;
      pk.x = uint32_t(f32_to_bf16(acc[0])) | (uint32_t(f32_to_bf16(acc[1])) << 16);
      pk.y = uint32_t(f32_to_bf16(acc[2])) | (uint32_t(f32_to_bf16(acc[3])) << 16);
      pk.z = uint32_t(f32_to_bf16(acc[4])) | (uint32_t(f32_to_bf16(acc[5])) << 16);
      pk.w = uint32_t(f32_to_bf16(acc[6])) | (uint32_t(f32_to_bf16(acc[7])) << 16);
      *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + t * ld_out + c) = pk;
    }
  }
}

// Unpermute with the router's share of the input gradient folded in (E <= 8):
//   out[t] = addend[t] + sum_k w[t,k] y[row_of[t,k]] + sum_e dl[t,e] W[e]
// i.e. the experts' and the router's input gradients of a MoE layer in one
// pass (no [T, D] router gradient written and read back).  Thread i of a
// workgroup owns columns 8 i .. 8 i + 8 of a 2048-column span (blockIdx.x)
// and keeps W's 8 x 8 values of them in registers; the workgroup walks the
// tokens [blockIdx.y * tpb, +tpb), four at a time with every load of the four
// issued before any use (KC = K when K is 1, 2 or 4, else 0 = a loop over
// K).  fp32 sums in the order addend, slots in order (separately rounded
// products and sums), then the router's terms; one rounding to the output
// dtype.
__device__ __forceinline__ void add_bf16x8(float (&acc)[8], uint4 pk, float s) {
#pragma clang fp contract(off)
  const uint32_t q[4] = {pk.x, pk.y, pk.z, pk.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    acc[2 * j] = acc[2 * j] + s * u2f(q[j] << 16);
    acc[2 * j + 1] = acc[2 * j + 1] + s * u2f(q[j] & 0xffff0000u);
  }
}

template <typename WT, int KC>
__global__ __launch_bounds__(256) void unpermute_router_kernel(const uint16_t* __restrict__ y, int64_t ld_y,
                                                               const int32_t* __restrict__ row_of,
                                                               const float* __restrict__ w,
                                                               int64_t T, int K, int64_t D,
                                                               void* __restrict__ out, int out_f32, int64_t ld_out,
                                                               const uint16_t* __restrict__ addend, int64_t ld_add,
                                                               const float* __restrict__ dl, int64_t ld_dl,
                                                               int dl_vec, const WT* __restrict__ W, int64_t ld_w,
                                                               int E, int64_t tpb) {
  const int64_t c = int64_t(blockIdx.x) * 2048 + threadIdx.x * 8;
  if (c >= D) return;
  // the gate's columns of this thread for the 8 experts, kept as stored
  // (bf16 packed in 32 registers, widened where used; fp32 in 64)
  constexpr int WW = sizeof(WT) == 2 ? 4 : 8;
  uint32_t wr[8][WW];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if (e < E) {
      const uint4* p = reinterpret_cast<const uint4*>(W + e * ld_w + c);
#pragma unroll
      for (int h = 0; h < WW / 4; ++h) {
        const uint4 q = p[h];
        wr[e][4 * h] = q.x; wr[e][4 * h + 1] = q.y; wr[e][4 * h + 2] = q.z; wr[e][4 * h + 3] = q.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < WW; ++j) wr[e][j] = 0u;
    }
  }
  auto w_row = [&](int e, float (&v)[8]) {
    if constexpr (sizeof(WT) == 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // opaque to the optimiser, so the widening stays here instead of being
        // hoisted out of the token loop into 64 live registers
        asm volatile("" : "+v"(wr[e][j]));
        v[2 * j] = u2f(wr[e][j] << 16);
        v[2 * j + 1] = u2f(wr[e][j] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = u2f(wr[e][j]);
    }
  };
  const int64_t t0 = int64_t(blockIdx.y) * tpb;
  const int64_t t1 = t0 + tpb < T ? t0 + tpb : T;
  for (int64_t tb = t0; tb < t1; tb += 4) {
    constexpr int KS = KC > 0 ? KC : 1;
    float acc[4][8];
    int32_t r[4][KS];
    float sw[4][KS];
    uint4 yv[4][KS];
    float d[4][8];
    // every load of the four tokens first (a token past t1 re-reads t1 - 1)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t t = tb + u < t1 ? tb + u : t1 - 1;
      if constexpr (KC > 0) {
#pragma unroll
        for (int k = 0; k < KC; ++k) {
          r[u][k] = row_of[t * KC + k];
          sw[u][k] = w ? w[t * KC + k] : 1.f;
        }
      }
      if (dl_vec) {   // E == 8, 16-byte aligned rows: the token's 8 dlogits as two 16-byte loads
        const float4 p0 = *reinterpret_cast<const float4*>(dl + t * ld_dl);
        const float4 p1 = *reinterpret_cast<const float4*>(dl + t * ld_dl + 4);
        d[u][0] = p0.x; d[u][1] = p0.y; d[u][2] = p0.z; d[u][3] = p0.w;
        d[u][4] = p1.x; d[u][5] = p1.y; d[u][6] = p1.z; d[u][7] = p1.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) d[u][e] = e < E ? dl[t * ld_dl + e] : 0.f;
      }
      if (addend) {
        const uint4 pk = *reinterpret_cast<const uint4*>(addend + t * ld_add + c);
        const uint32_t q[4] = {pk.x, pk.y, pk.z, pk.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[u][2 * j] = u2f(q[j] << 16);
          acc[u][2 * j + 1] = u2f(q[j] & 0xffff0000u);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[u][j] = 0.f;
      }
    }
    if constexpr (KC > 0) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int k = 0; k < KC; ++k)
          yv[u][k] = *reinterpret_cast<const uint4*>(y + int64_t(r[u][k] >= 0 ? r[u][k] : 0) * ld_y + c);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int k = 0; k < KC; ++k)
          if (r[u][k] >= 0) add_bf16x8(acc[u], yv[u][k], sw[u][k]);
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t t = tb + u < t1 ? tb + u : t1 - 1;
        for (int k = 0; k < K; ++k) {
          const int32_t rr = row_of[t * K + k];
          if (rr < 0) continue;
          add_bf16x8(acc[u], *reinterpret_cast<const uint4*>(y + int64_t(rr) * ld_y + c), w ? w[t * K + k] : 1.f);
        }
      }
    }
    // router term: sum over experts in expert order, after the slots' sum
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float wv[8];
      w_row(e, wv);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[u][j] = fmaf(d[u][e], wv[j], acc[u][j]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (tb + u >= t1) break;
      const int64_t t = tb + u;
      if (out_f32) {
        float* o = static_cast<float*>(out) + t * ld_out + c;
        *reinterpret_cast<float4*>(o) = make_float4(acc[u][0], acc[u][1], acc[u][2], acc[u][3]);
        *reinterpret_cast<float4*>(o + 4) = make_float4(acc[u][4], acc[u][5], acc[u][6], acc[u][7]);
      } else {
        uint4 pk;
        pk.x = hw_bf16x2(acc[u][0], acc[u][1]);
        pk.y = hw_bf16x2(acc[u][2], acc[u][3]);
        pk.z = hw_bf16x2(acc[u][4], acc[u][5]);
        pk.w = hw_bf16x2(acc[u][6], acc[u][7]);
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + t * ld_out + c) = pk;
      }
    }
  }
}

// one wave per assignment: dw[a] = sum_d dout[t][d] * y[row_of[a]][d], four
// 512-column chunks' loads issued before their products (summed in column
// order, as one chunk at a time would)
__global__ __launch_bounds__(256) void router_grad_kernel(const uint16_t* __restrict__ dout, int64_t ld_do,
                                                          const uint16_t* __restrict__ y, int64_t ld_y,
                                                          const int32_t* __restrict__ row_of, int64_t A, int K,
                                                          int64_t D, float* __restrict__ dw) {
  const int lane = threadIdx.x & 63;
  for (int64_t a = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6); a < A;
       a += int64_t(gridDim.x) * 4) {
    const int32_t r = row_of[a];
    float acc = 0.f;
    if (r >= 0) {
      const uint16_t* g = dout + (a / K) * ld_do;
      const uint16_t* yy = y + int64_t(r) * ld_y;
      for (int64_t c0 = int64_t(lane) * 8; c0 < D; c0 += 4 * 512) {
        uint4 p[4], q[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int64_t c = c0 + 512 * u;
          p[u] = c < D ? *reinterpret_cast<const uint4*>(g + c) : make_uint4(0, 0, 0, 0);
          q[u] = c < D ? *reinterpret_cast<const uint4*>(yy + c) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (c0 + 512 * u >= D) break;
          const uint32_t pw[4] = {p[u].x, p[u].y, p[u].z, p[u].w}, qw[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc += u2f(pw[j] << 16) * u2f(qw[j] << 16);
            acc += u2f(pw[j] & 0xffff0000u) * u2f(qw[j] & 0xffff0000u);
          }
        }
      }
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (lane == 0) dw[a] = acc;
  }
}

// ----------------------------------------------------- sort launcher ----
// Small sorts take the fused scan + scatter unless FM_ROUTE_FUSED_SCAN=0
// (read once).
inline bool gemm_route_fused_scan() {
  static const bool on = [] {
    const char* e = getenv("FM_ROUTE_FUSED_SCAN");
    return e == nullptr || atoi(e) != 0;
  }();
  return on;
}

// The sort kernels on one stream: histograms, then the scan and the scatter
// (one launch for small sorts).  block_hist ([E][blocks] int32) is written in
// full by sort_hist_kernel before anything reads it, so the buffer needs no
// clearing.
// Shares (percent of an expert-weight batch's blocks) that the histogram and
// the fused scan + scatter launches run beside their own workgroups
// (FM_SORT_SIDE="hist,scan", read once; without the fused launch the
// histogram takes both); the rest runs as its own launch.  Default: all in
// the fused launch -- one ramp and one tail for the whole batch, and the
// longer of the two sort launches hidden.
inline void sort_side_shares(int& hist, int& scan) {
  static const std::pair<int, int> v = [] {
    int h = 0, c = 100;
    if (const char* e = getenv("FM_SORT_SIDE")) sscanf(e, "%d,%d", &h, &c);
    h = h < 0 ? 0 : h > 100 ? 100 : h;
    c = c < 0 ? 0 : c > 100 - h ? 100 - h : c;
    return std::make_pair(h, c);
  }();
  hist = v.first;
  scan = v.second;
}

static int route_sort_launch(const void* indices, int indices_i64, int64_t T, int K, int E,
                             int64_t threshold, int32_t* counts, int32_t* offsets, int32_t* row_of,
                             int32_t* assign_of_row, int64_t rows_max, int32_t* tile_expert,
                             int32_t* use_fp8, int32_t* bh, hipStream_t sm, const char* what,
                             const WeightSide* side = nullptr) {
  const int64_t A = T * K;
  FM_REQUIRE(indices || A == 0, "%s: null indices", what);
  FM_REQUIRE(E >= 1 && E <= kSortMaxExperts, "%s: E must be in [1, %d]", what, kSortMaxExperts);
  FM_REQUIRE(counts && offsets && assign_of_row && tile_expert && (row_of || A == 0), "%s: null output", what);
  FM_REQUIRE(rows_max >= fm_route_rows_max(A, E) && rows_max % 128 == 0,
             "%s: rows_max must be >= fm_route_rows_max() and a multiple of 128", what);
  const int64_t nb = (A + kSortBlock - 1) / kSortBlock;
  const bool fused = nb > 0 && nb <= kFusedBlocks && E <= kFusedExperts && gemm_route_fused_scan();
  // weight blocks: [0, wh) beside the histograms, [wh, wh + ws) beside the
  // fused scan + scatter, the rest on their own after the sort
  WeightSide sh{}, sc{};
  int64_t wh = 0, wsc = 0;
  if (side != nullptr && nb > 0) {
    int ph, pc;
    sort_side_shares(ph, pc);
    wh = side->total * (fused ? ph : ph + pc) / 100;
    wsc = fused ? side->total * pc / 100 : 0;
    sh = *side;
    sh.first = 0;
    sh.count = wh;
    sc = *side;
    sc.first = wh;
    sc.count = wsc;
    FM_REQUIRE(nb + wh < (int64_t(1) << 31) && nb + wsc < (int64_t(1) << 31), "%s: too many weight blocks", what);
  }
  if (nb > 0) {
    const dim3 g(unsigned(nb + wh));
    if (indices_i64)
      hipLaunchKernelGGL(sort_hist_kernel<int64_t>, g, dim3(256), 0, sm, static_cast<const int64_t*>(indices), A, E,
                         bh, nb, sh);
    else
      hipLaunchKernelGGL(sort_hist_kernel<int32_t>, g, dim3(256), 0, sm, static_cast<const int32_t*>(indices), A, E,
                         bh, nb, sh);
    if (int rc = check_launch(what)) return rc;
  }
  auto rest = [&]() -> int {
    return side != nullptr ? launch_weight_side(*side, wh + wsc, side->total - wh - wsc, sm) : 0;
  };
  if (fused) {
    const dim3 g(unsigned(nb + wsc));
    if (indices_i64)
      hipLaunchKernelGGL(sort_scan_scatter_kernel<int64_t>, g, dim3(256), 0, sm,
                         static_cast<const int64_t*>(indices), A, E, bh, nb, counts, offsets, tile_expert,
                         rows_max / 128, row_of, assign_of_row, rows_max, use_fp8, threshold, sc);
    else
      hipLaunchKernelGGL(sort_scan_scatter_kernel<int32_t>, g, dim3(256), 0, sm,
                         static_cast<const int32_t*>(indices), A, E, bh, nb, counts, offsets, tile_expert,
                         rows_max / 128, row_of, assign_of_row, rows_max, use_fp8, threshold, sc);
    if (int rc = check_launch(what)) return rc;
    return rest();
  }
  hipLaunchKernelGGL(sort_scan_kernel, dim3(1), dim3(1024), 0, sm, bh, nb, E, counts, offsets,
                     tile_expert, rows_max / 128, assign_of_row, rows_max, use_fp8, threshold);
  if (int rc = check_launch(what)) return rc;
  if (nb > 0) {
    if (indices_i64)
      hipLaunchKernelGGL(sort_scatter_kernel<int64_t>, dim3(unsigned(nb)), dim3(256), 0, sm,
                         static_cast<const int64_t*>(indices), A, E, bh, nb, offsets, row_of,
                         assign_of_row);
    else
      hipLaunchKernelGGL(sort_scatter_kernel<int32_t>, dim3(unsigned(nb)), dim3(256), 0, sm,
                         static_cast<const int32_t*>(indices), A, E, bh, nb, offsets, row_of,
                         assign_of_row);
    if (int rc = check_launch(what)) return rc;
  }
  return rest();
}

// ------------------------------------------------ allocation-free scratch ----
// The block histogram of fm_route_sort_noalloc lives in this fixed device
// array (one copy per GPU, held until the process ends).  Host code never
// passes `scratch` itself to a kernel: its device address is looked up once
// per device with hipGetSymbolAddress and cached below.  Every call on a GPU
// shares that GPU's array, so calls that overlap on one GPU (two streams, two
// host threads) race; calls ordered on one stream do not.
constexpr int64_t kRouteScratchBytes = int64_t(2) << 20;   // 2 MiB: E * ceil(A / 1024) <= 524288
static __device__ __align__(256) uint8_t scratch[kRouteScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static int32_t* g_scratch_ptr[kMaxDevices] = {};

static int route_scratch_ptr(int32_t** out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  FM_REQUIRE(err == hipSuccess, "fm_route_sort_noalloc: hipGetDevice failed: %s", hipGetErrorString(err));
  FM_REQUIRE(dev >= 0 && dev < kMaxDevices, "fm_route_sort_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    FM_REQUIRE(err == hipSuccess && p, "fm_route_sort_noalloc: hipGetSymbolAddress(scratch) failed: %s",
               hipGetErrorString(err));
    g_scratch_ptr[dev] = static_cast<int32_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return 0;
}


// ------------------------------------------------------------- capacity ----
// Token dropping by expert capacity.  An expert's tokens are ranked in token
// order; a token is kept when each of its valid slots ranks below the
// capacity.  The stable sort puts each expert's assignments in token order
// (assignment a = t*K + k, and the K experts of a token are distinct), so a
// slot's rank is its row less its group's start.
constexpr int kCapBlock = 1024;   // tokens per workgroup (256 threads x 4)

// pos_of[t] = 0 (kept) or -1 (dropped); block_kept[b] = kept tokens of
// workgroup b.  Workgroup 0 also writes drops[e] = max(0, counts[e] -
// capacity).
template <typename I>
__global__ __launch_bounds__(256) void capacity_keep_kernel(const I* __restrict__ idx, int64_t T, int K, int E,
                                                            const int32_t* __restrict__ counts,
                                                            const int32_t* __restrict__ offsets,
                                                            const int32_t* __restrict__ row_of, int64_t capacity,
                                                            int32_t* __restrict__ pos_of,
                                                            int32_t* __restrict__ block_kept,
                                                            int32_t* __restrict__ drops) {
  int kept = 0;
#pragma unroll 1
  for (int i = 0; i < kCapBlock / 256; ++i) {
    const int64_t t = int64_t(blockIdx.x) * kCapBlock + i * 256 + threadIdx.x;
    int keep = 0;
    if (t < T) {
      keep = 1;
      for (int k = 0; k < K; ++k) {
        const int64_t a = t * K + k;
        const int e = load_expert(idx, a, E);
        const int32_t r = row_of[a];
        if (e >= 0 && r >= 0 && int64_t(r - offsets[e]) >= capacity) keep = 0;
      }
      st_global(reinterpret_cast<uint32_t*>(pos_of + t), uint32_t(keep ? 0 : -1));
    }
    kept += __syncthreads_count(keep);
  }
  if (threadIdx.x == 0) st_global(reinterpret_cast<uint32_t*>(block_kept + blockIdx.x), uint32_t(kept));
  if (blockIdx.x == 0)
    for (int e = threadIdx.x; e < E; e += 256) {
      const int64_t over = int64_t(counts[e]) - capacity;
      st_global(reinterpret_cast<uint32_t*>(drops + e), uint32_t(over > 0 ? over : 0));
    }
}

// Compaction: workgroup b starts at the kept tokens of the workgroups before
// it, then ranks its own with wave ballots.  pos_of[t] becomes the token's
// position among the kept ones (or stays -1), kept_index[pos] = t, and the
// last workgroup writes the total to n_kept.
__global__ __launch_bounds__(256) void capacity_compact_kernel(int64_t T, const int32_t* __restrict__ block_kept,
                                                               int64_t n_blocks, int32_t* __restrict__ pos_of,
                                                               int32_t* __restrict__ kept_index,
                                                               int32_t* __restrict__ n_kept) {
  __shared__ int32_t part[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int32_t before = 0;
  for (int64_t j = threadIdx.x; j < int64_t(blockIdx.x); j += 256) before += block_kept[j];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) before += __shfl_xor(before, off);
  if (lane == 0) part[wave] = before;
  __syncthreads();
  int32_t base = part[0] + part[1] + part[2] + part[3];
  __syncthreads();
#pragma unroll 1
  for (int i = 0; i < kCapBlock / 256; ++i) {
    const int64_t t = int64_t(blockIdx.x) * kCapBlock + i * 256 + threadIdx.x;
    const bool keep = t < T && pos_of[t] >= 0;
    const uint64_t m = __ballot(keep);
    if (lane == 0) part[wave] = __popcll(m);
    __syncthreads();
    int32_t pos = base + __popcll(m & lanemask_lt());
    for (int w = 0; w < wave; ++w) pos += part[w];
    if (keep) {
      st_global(reinterpret_cast<uint32_t*>(pos_of + t), uint32_t(pos));
      st_global(reinterpret_cast<uint32_t*>(kept_index + pos), uint32_t(t));
    }
    base += part[0] + part[1] + part[2] + part[3];
    __syncthreads();
  }
  if (int64_t(blockIdx.x) == n_blocks - 1 && threadIdx.x == 0) st_global(reinterpret_cast<uint32_t*>(n_kept),
                                                                          uint32_t(base));
}

// dst row i = src row index[i], zeros where index[i] is outside [0, n_src).
// VW-byte pieces (16 or 4), a piece per thread, rows walked by the grid.
template <int VW>
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint8_t* __restrict__ src, int64_t n_src,
                                                          int64_t ld_src, const int32_t* __restrict__ index,
                                                          int64_t n, int64_t pieces, uint8_t* __restrict__ dst,
                                                          int64_t ld_dst) {
  using V = typename std::conditional<VW == 16, uint4, uint32_t>::type;
  const int64_t total = n * pieces;
  for (int64_t q = int64_t(blockIdx.x) * 256 + threadIdx.x; q < total; q += int64_t(gridDim.x) * 256) {
    const int64_t i = q / pieces, c = q - i * pieces;
    const int64_t r = index[i];
    V v{};
    if (r >= 0 && r < n_src) v = *reinterpret_cast<const V*>(src + r * ld_src + c * VW);
    st_global(reinterpret_cast<V*>(dst + i * ld_dst + c * VW), v);
  }
}

}  // namespace fm

using namespace fm;

extern "C" {

int fm_topk_gating(const float* logits, int64_t T, int E, int64_t ld, int K, int gating, int flags,
                   const void* replay_indices, int replay_i64, float* weights, void* indices, int indices_i64,
                   float* prob_partial, float* z_partial, int64_t n_waves, void* stream) {
  FM_REQUIRE(logits && weights && indices, "fm_topk_gating: null pointer");
  FM_REQUIRE(E >= 1 && E <= 64 * kTopkMaxPerLane, "fm_topk_gating: E must be in [1, %d] (got %d)",
             64 * kTopkMaxPerLane, E);
  FM_REQUIRE(K >= 1 && K <= E && K <= 64, "fm_topk_gating: K must be in [1, min(E, 64)] (got %d)", K);
  FM_REQUIRE(gating == FM_GATING_SOFTMAX || gating == FM_GATING_SIGMOID, "fm_topk_gating: bad gating");
  FM_REQUIRE((flags & ~FM_GATING_L2_NORMALIZE) == 0, "fm_topk_gating: unknown flags 0x%x", flags);
  FM_REQUIRE(ld >= E, "fm_topk_gating: pitch < E");
  FM_REQUIRE(n_waves >= 4 && n_waves % 4 == 0, "fm_topk_gating: n_waves must be a positive multiple of 4");
  if (T == 0) return 0;
  TopkArgs a{logits, T, ld, E, K, gating == FM_GATING_SIGMOID, (flags & FM_GATING_L2_NORMALIZE) ? 1 : 0,
             replay_indices, replay_i64, weights, indices, indices_i64, prob_partial, z_partial};
  const dim3 grid(unsigned(n_waves / 4)), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (E <= 2) hipLaunchKernelGGL(topk_small_kernel<2>, grid, block, 0, s, a);
  else if (E <= 4) hipLaunchKernelGGL(topk_small_kernel<4>, grid, block, 0, s, a);
  else if (E <= 8) hipLaunchKernelGGL(topk_small_kernel<8>, grid, block, 0, s, a);
  else if (E <= 16) hipLaunchKernelGGL(topk_small_kernel<16>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(topk_kernel, grid, block, 0, s, a);
  return check_launch("fm_topk_gating");
}

int fm_aux_loss(const float* prob_partial, int64_t n_waves, const int32_t* counts, int E, int64_t T,
                const float* z_partial, float z_loss_multiplier, float* loss, void* stream) {
  FM_REQUIRE(prob_partial && counts && loss, "fm_aux_loss: null pointer");
  FM_REQUIRE(T > 0 && E > 0 && E <= 1024, "fm_aux_loss: T must be positive and E in [1, 1024] (got %d)", E);
  hipLaunchKernelGGL(aux_loss_kernel, dim3(1), dim3(512), 0, static_cast<hipStream_t>(stream),
                     prob_partial, n_waves, counts, E, T, z_partial, z_loss_multiplier, loss);
  return check_launch("fm_aux_loss");
}

// sum_e ceil(n_e / 128) <= sum_e (n_e + 127) / 128 = (A + 127 E) / 128, an
// integer, so the padded groups fit in floor((A + 127 E) / 128) tiles (E = 1:
// exactly ceil(A / 128)); at least one tile.
int64_t fm_route_rows_max(int64_t assignments, int E) {
  const int64_t tiles = (assignments + int64_t(E) * 127) / 128;
  return (tiles > 0 ? tiles : 1) * 128;
}

int64_t fm_route_workspace_bytes(int64_t assignments, int E) {
  const int64_t nb = (assignments + kSortBlock - 1) / kSortBlock;
  return (nb > 0 ? nb : 1) * E * int64_t(sizeof(int32_t));
}

int fm_route_sort(const void* indices, int indices_i64, int64_t T, int K, int E,
                  int64_t threshold, int32_t* counts, int32_t* offsets, int32_t* row_of,
                  int32_t* assign_of_row, int64_t rows_max, int32_t* tile_expert,
                  int32_t* use_fp8, void* workspace, int64_t workspace_bytes, void* stream) {
  FM_REQUIRE(workspace, "fm_route_sort: null workspace");
  FM_REQUIRE(workspace_bytes >= fm_route_workspace_bytes(T * K, E), "fm_route_sort: workspace too small");
  return route_sort_launch(indices, indices_i64, T, K, E, threshold, counts, offsets, row_of, assign_of_row,
                           rows_max, tile_expert, use_fp8, static_cast<int32_t*>(workspace),
                           static_cast<hipStream_t>(stream), "fm_route_sort");
}

int fm_route_sort_weights(const void* indices, int indices_i64, int64_t T, int K, int E, int64_t threshold,
                          int32_t* counts, int32_t* offsets, int32_t* row_of, int32_t* assign_of_row,
                          int64_t rows_max, int32_t* tile_expert, int32_t* use_fp8, void* workspace,
                          int64_t workspace_bytes, const FmWeightJob* jobs, int n_jobs, void* stream) {
  FM_REQUIRE(workspace, "fm_route_sort_weights: null workspace");
  FM_REQUIRE(workspace_bytes >= fm_route_workspace_bytes(T * K, E), "fm_route_sort_weights: workspace too small");
  WeightSide side;
  if (int rc = make_weight_side(jobs, n_jobs, side, "fm_route_sort_weights")) return rc;
  return route_sort_launch(indices, indices_i64, T, K, E, threshold, counts, offsets, row_of, assign_of_row,
                           rows_max, tile_expert, use_fp8, static_cast<int32_t*>(workspace),
                           static_cast<hipStream_t>(stream), "fm_route_sort_weights", &side);
}

int64_t fm_route_sort_noalloc_max_workspace_bytes(void) { return kRouteScratchBytes; }

int fm_route_sort_noalloc(const void* indices, int indices_i64, int64_t T, int K, int E,
                          int64_t threshold, int32_t* counts, int32_t* offsets, int32_t* row_of,
                          int32_t* assign_of_row, int64_t rows_max, int32_t* tile_expert,
                          int32_t* use_fp8, void* stream) {
  FM_REQUIRE(E >= 1 && E <= kSortMaxExperts, "fm_route_sort_noalloc: E must be in [1, %d]", kSortMaxExperts);
  FM_REQUIRE(T >= 0 && K >= 1, "fm_route_sort_noalloc: T must be >= 0 and K >= 1");
  const int64_t need = fm_route_workspace_bytes(T * K, E);
  FM_REQUIRE(need <= kRouteScratchBytes,
             "fm_route_sort_noalloc: %lld assignments over %d experts need %lld bytes of scratch, more than "
             "the %lld this entry point holds (use fm_route_sort with a workspace)",
             (long long)(T * K), E, (long long)need, (long long)kRouteScratchBytes);
  int32_t* bh = nullptr;
  if (int rc = route_scratch_ptr(&bh)) return rc;
  return route_sort_launch(indices, indices_i64, T, K, E, threshold, counts, offsets, row_of, assign_of_row,
                           rows_max, tile_expert, use_fp8, bh, static_cast<hipStream_t>(stream),
                           "fm_route_sort_noalloc");
}

int fm_route_tile_masks(const int32_t* tile_expert, int64_t n_tiles, const int32_t* use_fp8, int32_t* tiles_fp8,
                        int32_t* tiles_bf16, void* stream) {
  FM_REQUIRE((tile_expert && use_fp8 && tiles_fp8 && tiles_bf16) || n_tiles == 0,
             "fm_route_tile_masks: null pointer");
  FM_REQUIRE(n_tiles >= 0, "fm_route_tile_masks: n_tiles must be >= 0");
  if (n_tiles == 0) return 0;
  const unsigned blocks = unsigned((n_tiles + 255) / 256 < 1024 ? (n_tiles + 255) / 256 : 1024);
  hipLaunchKernelGGL(tile_masks_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), tile_expert,
                     n_tiles, use_fp8, tiles_fp8, tiles_bf16);
  return check_launch("fm_route_tile_masks");
}

int fm_permute(const void* x, int64_t T, int64_t D, int64_t ld_x, const int32_t* assign_of_row,
               int64_t rows, int K, const float* weights, int kind, void* q, int64_t ld_q, void* s,
               int64_t ld_s, void* qt, int64_t ld_qt, void* st, int64_t ld_st,
               const int32_t* tile_valid, void* stream) {
  FM_REQUIRE(x || T == 0, "fm_permute: null input");
  FM_REQUIRE(assign_of_row, "fm_permute: null assign_of_row");
  FM_REQUIRE(ld_x >= D && ld_x % 8 == 0, "fm_permute: input pitch must be >= D and a multiple of 8");
  FM_REQUIRE(K >= 1, "fm_permute: K must be >= 1");
  const TileOut o = make_tile_out(kind, q, ld_q, s, ld_s, qt, ld_qt, st, ld_st, 0, 0, tile_valid);
  const hipStream_t sm = static_cast<hipStream_t>(stream);
  if (T == 0) return launch_tile_producer(ZeroSrc{}, o, rows, D, sm, "fm_permute");
  const uint16_t* xs = static_cast<const uint16_t*>(x);
  if (weights) return launch_tile_producer(GatherSrc<true>{xs, ld_x, assign_of_row, K, weights}, o, rows, D, sm,
                                           "fm_permute");
  return launch_tile_producer(GatherSrc<false>{xs, ld_x, assign_of_row, K, nullptr}, o, rows, D, sm,
                              "fm_permute");
}

int fm_unpermute(const void* y, int64_t ld_y, const int32_t* row_of, const float* weights,
                 int64_t T, int K, int64_t D, void* out, int out_dtype, int64_t ld_out,
                 const void* addend, int64_t ld_add, void* stream) {
  FM_REQUIRE((y && row_of && out) || T == 0, "fm_unpermute: null pointer");
  FM_REQUIRE(D % 8 == 0 && ld_y % 8 == 0 && ld_out % 8 == 0 && (addend == nullptr || ld_add % 8 == 0),
             "fm_unpermute: D and pitches must be multiples of 8");
  FM_REQUIRE(out_dtype == FM_DTYPE_BF16 || out_dtype == FM_DTYPE_F32, "fm_unpermute: bad out dtype");
  FM_REQUIRE(aligned16(y) && aligned16(out) && aligned16(addend),
             "fm_unpermute: y, out and addend must be 16-byte aligned (8-element vector accesses)");
  if (T == 0) return 0;
  const int64_t n = T * (D / 8);
  const unsigned blocks = unsigned(n / 256 + 1 < 16384 ? n / 256 + 1 : 16384);
  // slot indices and weights as vectors when their rows are 16-byte aligned
  // (K = 4, 8; K = 8 with one local slot per token at D = 7168: 399 -> 361 us)
  const bool vec = (K == 4 || K == 8) && aligned16(row_of) && aligned16(weights);
  auto go = [&](auto kc) {
    constexpr int KC = decltype(kc)::value;
    if constexpr (KC == 4 || KC == 8) {
      if (vec) {
        hipLaunchKernelGGL((unpermute_kernel<KC, true>), dim3(blocks), dim3(256), 0,
                           static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(y), ld_y, row_of, weights,
                           T, K, D, out, out_dtype == FM_DTYPE_F32, ld_out, static_cast<const uint16_t*>(addend),
                           ld_add);
        return;
      }
    }
    hipLaunchKernelGGL((unpermute_kernel<KC>), dim3(blocks), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(y), ld_y, row_of, weights,
                       T, K, D, out, out_dtype == FM_DTYPE_F32, ld_out, static_cast<const uint16_t*>(addend),
                       ld_add);
  };
  if (K == 1) go(std::integral_constant<int, 1>{});
  else if (K == 2) go(std::integral_constant<int, 2>{});
  else if (K == 4) go(std::integral_constant<int, 4>{});
  else if (K == 8) go(std::integral_constant<int, 8>{});
  else go(std::integral_constant<int, 0>{});
  return check_launch("fm_unpermute");
}

int fm_unpermute_router(const void* y, int64_t ld_y, const int32_t* row_of, const float* weights,
                        int64_t T, int K, int64_t D, void* out, int out_dtype, int64_t ld_out,
                        const void* addend, int64_t ld_add, const float* dlogits, int64_t ld_dl,
                        const void* gate_w, int gate_dtype, int64_t ld_w, int E, void* stream) {
  FM_REQUIRE((y && row_of && out && dlogits && gate_w) || T == 0, "fm_unpermute_router: null pointer");
  FM_REQUIRE(E >= 1 && E <= 8, "fm_unpermute_router: E must be in [1, 8] (got %d)", E);
  FM_REQUIRE(D % 8 == 0 && ld_y % 8 == 0 && ld_out % 8 == 0 && ld_w % 8 == 0 &&
                 (addend == nullptr || ld_add % 8 == 0) && ld_dl >= E,
             "fm_unpermute_router: D and pitches must be multiples of 8");
  FM_REQUIRE(out_dtype == FM_DTYPE_BF16 || out_dtype == FM_DTYPE_F32, "fm_unpermute_router: bad out dtype");
  FM_REQUIRE(gate_dtype == FM_DTYPE_BF16 || gate_dtype == FM_DTYPE_F32, "fm_unpermute_router: bad gate dtype");
  FM_REQUIRE(aligned16(y) && aligned16(out) && aligned16(addend) && aligned16(gate_w),
             "fm_unpermute_router: y, out, addend and gate_w must be 16-byte aligned (8-element vector accesses)");
  if (T == 0) return 0;
  const int dl_vec = E == 8 && ld_dl % 4 == 0 && aligned16(dlogits) ? 1 : 0;
  const int64_t nx = (D + 2047) / 2048;
  hipStream_t sm = static_cast<hipStream_t>(stream);
  auto go = [&](auto wt, auto kc) {
    using WT = decltype(wt);
    // as many workgroups as fit at once (one round: a partly filled second
    // round measured 26 against 23 us at configs[2]), each a run of tokens
    static const int64_t nwg = resident_workgroups(unpermute_router_kernel<WT, decltype(kc)::value>, 256);
    int64_t tpb = (T * nx + nwg - 1) / nwg;
    if (tpb < 1) tpb = 1;
    const dim3 grid(unsigned(nx), unsigned((T + tpb - 1) / tpb));
    hipLaunchKernelGGL((unpermute_router_kernel<WT, decltype(kc)::value>), grid, dim3(256), 0, sm,
                       static_cast<const uint16_t*>(y), ld_y, row_of, weights, T, K, D, out,
                       out_dtype == FM_DTYPE_F32, ld_out, static_cast<const uint16_t*>(addend), ld_add, dlogits,
                       ld_dl, dl_vec, static_cast<const WT*>(gate_w), ld_w, E, tpb);
  };
  auto go_k = [&](auto wt) {
    if (K == 1) go(wt, std::integral_constant<int, 1>{});
    else if (K == 2) go(wt, std::integral_constant<int, 2>{});
    else if (K == 4) go(wt, std::integral_constant<int, 4>{});
    else go(wt, std::integral_constant<int, 0>{});
  };
  if (gate_dtype == FM_DTYPE_F32) go_k(float{});
  else go_k(uint16_t{});
  return check_launch("fm_unpermute_router");
}

int fm_router_weight_grad(const void* dout, int64_t ld_do, const void* y, int64_t ld_y,
                          const int32_t* row_of, int64_t T, int K, int64_t D, float* dw,
                          void* stream) {
  FM_REQUIRE((dout && y && row_of && dw) || T == 0, "fm_router_weight_grad: null pointer");
  FM_REQUIRE(D % 8 == 0 && ld_do % 8 == 0 && ld_y % 8 == 0,
             "fm_router_weight_grad: D and pitches must be multiples of 8");
  if (T == 0) return 0;
  const int64_t A = T * K;
  const unsigned blocks = unsigned(A / 4 + 1 < 16384 ? A / 4 + 1 : 16384);
  hipLaunchKernelGGL(router_grad_kernel, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(dout), ld_do,
                     static_cast<const uint16_t*>(y), ld_y, row_of, A, K, D, dw);
  return check_launch("fm_router_weight_grad");
}


int64_t fm_capacity_workspace_bytes(int64_t T) {
  const int64_t blocks = T <= 0 ? 1 : (T + kCapBlock - 1) / kCapBlock;
  return (blocks * 4 + 255) / 256 * 256;
}

int fm_capacity_select(const void* indices, int indices_i64, int64_t T, int K, int E, const int32_t* counts,
                       const int32_t* offsets, const int32_t* row_of, int64_t capacity, int32_t* pos_of,
                       int32_t* kept_index, int32_t* n_kept, int32_t* drops, void* workspace,
                       int64_t workspace_bytes, void* stream) {
  FM_REQUIRE(T >= 0 && K >= 1 && E >= 1 && E <= kSortMaxExperts, "fm_capacity_select: bad T, K or E");
  FM_REQUIRE(T * K < (int64_t(1) << 31), "fm_capacity_select: T*K must be below 2^31");
  FM_REQUIRE(capacity >= 0, "fm_capacity_select: capacity must be >= 0");
  FM_REQUIRE(counts && offsets && n_kept && drops && (T == 0 || (indices && row_of && pos_of && kept_index)),
             "fm_capacity_select: null pointer");
  FM_REQUIRE(workspace && workspace_bytes >= fm_capacity_workspace_bytes(T),
             "fm_capacity_select: workspace must hold fm_capacity_workspace_bytes(T) bytes");
  hipStream_t sm = static_cast<hipStream_t>(stream);
  // (T == 0: one workgroup of each kernel writes n_kept = 0 and the drops)
  const int64_t blocks = T == 0 ? 1 : (T + kCapBlock - 1) / kCapBlock;
  int32_t* bk = static_cast<int32_t*>(workspace);
  if (indices_i64)
    hipLaunchKernelGGL(capacity_keep_kernel<int64_t>, dim3(unsigned(blocks)), dim3(256), 0, sm,
                       static_cast<const int64_t*>(indices), T, K, E, counts, offsets, row_of, capacity, pos_of, bk,
                       drops);
  else
    hipLaunchKernelGGL(capacity_keep_kernel<int32_t>, dim3(unsigned(blocks)), dim3(256), 0, sm,
                       static_cast<const int32_t*>(indices), T, K, E, counts, offsets, row_of, capacity, pos_of, bk,
                       drops);
  hipLaunchKernelGGL(capacity_compact_kernel, dim3(unsigned(blocks)), dim3(256), 0, sm, T, bk, blocks, pos_of,
                     kept_index, n_kept);
  return check_launch("fm_capacity_select");
}

int fm_gather_rows(const void* src, int64_t n_src, int64_t ld_src, const int32_t* index, int64_t n,
                   int64_t row_bytes, void* dst, int64_t ld_dst, void* stream) {
  FM_REQUIRE(n >= 0 && n_src >= 0 && row_bytes >= 0, "fm_gather_rows: sizes must be >= 0");
  FM_REQUIRE(row_bytes % 4 == 0 && ld_src % 4 == 0 && ld_dst % 4 == 0 && ld_src >= row_bytes && ld_dst >= row_bytes,
             "fm_gather_rows: row bytes and pitches must be multiples of 4, pitches >= row bytes");
  FM_REQUIRE((n == 0 || row_bytes == 0) || (index && dst && (src || n_src == 0)), "fm_gather_rows: null pointer");
  FM_REQUIRE(reinterpret_cast<uintptr_t>(src) % 4 == 0 && reinterpret_cast<uintptr_t>(dst) % 4 == 0,
             "fm_gather_rows: src and dst must be 4-byte aligned");
  if (n == 0 || row_bytes == 0) return 0;
  hipStream_t sm = static_cast<hipStream_t>(stream);
  const bool v16 = row_bytes % 16 == 0 && ld_src % 16 == 0 && ld_dst % 16 == 0 && aligned16(src) && aligned16(dst);
  const int vw = v16 ? 16 : 4;
  const int64_t pieces = row_bytes / vw, total = n * pieces;
  const unsigned blocks = unsigned((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
  const uint8_t* s8 = static_cast<const uint8_t*>(src);
  uint8_t* d8 = static_cast<uint8_t*>(dst);
  if (v16) hipLaunchKernelGGL(gather_rows_kernel<16>, dim3(blocks), dim3(256), 0, sm, s8, n_src, ld_src, index, n,
                              pieces, d8, ld_dst);
  else hipLaunchKernelGGL(gather_rows_kernel<4>, dim3(blocks), dim3(256), 0, sm, s8, n_src, ld_src, index, n,
                          pieces, d8, ld_dst);
  return check_launch("fm_gather_rows");
}

}  // extern "C"
