// Expert-weight quantisation in 128 x 128 blocks: the per-tile body shared by
// fm_quantize_weight_batch's own launch and by launches that run a share of a
// batch's blocks as extra workgroups beside their own (fm_route_sort_weights:
// the routing sort's few workgroups leave most CUs idle).
#pragma once
#include "fm_tile.h"
#include "../../include/fm_hip.h"

namespace fm {

// ------------------------------------------------------------------ sources ----
template <typename T>
struct DenseSrc;

template <>
struct DenseSrc<uint16_t> {
  static constexpr int kOut = 1;
  const uint16_t* p;
  int64_t ld;
  struct Raw {
    uint4 pk;
  };
  __device__ __forceinline__ Raw fetch(int64_t row, int64_t col) const {
    return Raw{*reinterpret_cast<const uint4*>(p + row * ld + col)};
  }
  __device__ __forceinline__ void compute(const Raw& r, float v[][8]) const { unpack8_bf16(r.pk, v[0]); }
  __device__ __forceinline__ void load8(int64_t row, int64_t col, float v[][8]) const { compute(fetch(row, col), v); }
};

template <>
struct DenseSrc<float> {
  static constexpr int kOut = 1;
  const float* p;
  int64_t ld;
  struct Raw {
    float4 a, b;
  };
  __device__ __forceinline__ Raw fetch(int64_t row, int64_t col) const {
    return Raw{*reinterpret_cast<const float4*>(p + row * ld + col),
               *reinterpret_cast<const float4*>(p + row * ld + col + 4)};
  }
  __device__ __forceinline__ void compute(const Raw& r, float v[][8]) const {
    v[0][0] = r.a.x; v[0][1] = r.a.y; v[0][2] = r.a.z; v[0][3] = r.a.w;
    v[0][4] = r.b.x; v[0][5] = r.b.y; v[0][6] = r.b.z; v[0][7] = r.b.w;
  }
  __device__ __forceinline__ void load8(int64_t row, int64_t col, float v[][8]) const { compute(fetch(row, col), v); }
};

// ------------------------------------------------------- 128x128 weight blocks ----
struct WeightQuantArgs {
  const void* w;       // [G][R][C] source, pitch ld_w, group stride gs_w (elements)
  int src_f32;
  int64_t ld_w, gs_w;
  int kind;            // QK_BF16 / QK_BLOCK / QK_POW2
  uint8_t* q;          // [G][.][C] e4m3 (or bf16 if kind == QK_BF16), rows offset q_row_off
  int64_t ld_q, gs_q, q_row_off;
  float* s;            // [G][./128][C/128]
  int64_t ld_s, gs_s;
  uint8_t* qt;         // [G][C][.] transposed payload, columns offset qt_col_off
  int64_t ld_qt, gs_qt, qt_col_off;
  float* st;           // [G][C/128][./128]
  int64_t ld_st, gs_st;
  int paired;          // e4m3 q in the paired-row layout (FM_ROWS_PAIRED)
};

// Tile (ty, tx) of group g; 256 threads.  Thread t loads rows rr + 16*i
// (rr = t/16, i < 8), columns [8*(t%16), +8) of the tile; the whole tile
// shares one scale.  The transposed payload is staged through LDS so each
// thread writes whole 16-byte pieces of a transposed row.
template <typename T>
__device__ __forceinline__ void weight_quant_tile(const WeightQuantArgs& a, int64_t g, int64_t ty, int64_t tx,
                                                  float (&red)[256], uint32_t (&tile)[128][65]) {
  const int tid = threadIdx.x;
  const int64_t r0 = ty * 128, c0 = tx * 128;
  const int cc = (tid & 15) * 8;
  const int rr = tid >> 4;
  const DenseSrc<T> src{static_cast<const T*>(a.w) + g * a.gs_w, a.ld_w};
  if (a.kind == QK_BF16) {
    // bf16 payload: a bf16 source's words copied as they are, fp32 rounded
    uint32_t wv[8][4];
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint4 q = *reinterpret_cast<const uint4*>(src.p + (r0 + rr + 16 * i) * src.ld + c0 + cc);
        wv[i][0] = q.x; wv[i][1] = q.y; wv[i][2] = q.z; wv[i][3] = q.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float vi[1][8];
        src.load8(r0 + rr + 16 * i, c0 + cc, vi);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          wv[i][j] = uint32_t(f32_to_bf16(vi[0][2 * j])) | (uint32_t(f32_to_bf16(vi[0][2 * j + 1])) << 16);
      }
    }
    uint16_t* q16 = reinterpret_cast<uint16_t*>(a.q);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = rr + 16 * i;
      const uint32_t (&w)[4] = wv[i];
      if (q16)
        *reinterpret_cast<uint4*>(q16 + g * a.gs_q + (r0 + row + a.q_row_off) * a.ld_q + c0 + cc) =
            make_uint4(w[0], w[1], w[2], w[3]);
      if (a.qt) {
#pragma unroll
        for (int j = 0; j < 4; ++j) tile[row][(cc >> 1) + j] = w[j];
      }
    }
    if (!a.qt) return;
    __syncthreads();
    // transposed payload: 16 lanes per transposed row (256 bytes: the tile's
    // 128 rows of one column), lane k taking tile rows [8 k, 8 k + 8), so
    // each store instruction writes 4 whole rows of the transpose
    uint16_t* const base = reinterpret_cast<uint16_t*>(a.qt) + g * a.gs_qt + a.qt_col_off + r0;
    const int k = tid & 15;
#pragma unroll
    for (int pass = 0; pass < 8; ++pass) {
      const int col = pass * 16 + (tid >> 4);
      uint32_t w4[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int row = 8 * k + 2 * m;
        const uint32_t lo = (tile[row][col >> 1] >> (16 * (col & 1))) & 0xffffu;
        const uint32_t hi = (tile[row + 1][col >> 1] >> (16 * (col & 1))) & 0xffffu;
        w4[m] = lo | (hi << 16);
      }
      *reinterpret_cast<uint4*>(base + (c0 + col) * a.ld_qt + 8 * k) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    }
    return;
  }
  float v[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i) src.load8(r0 + rr + 16 * i, c0 + cc, v + i);
  float am = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) am = fmaxf(am, fabsf(v[i][j]));
  // block amax: wave maximum, then the four waves' through LDS
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) am = fmaxf(am, __shfl_xor(am, off));
  if ((tid & 63) == 0) red[tid >> 6] = am;
  __syncthreads();
  const float s = block_scale_dev(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), a.kind == QK_POW2);
  const bool pow2 = a.kind == QK_POW2;
  const float inv = pow2 ? pow2_recip(s) : 0.f;  // exact for power-of-two scales
  const Recip d = recip_of(s);
  constexpr bool HW = FM_HW_CVT != 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = rr + 16 * i;
    float f[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = pow2 ? v[i][j] * inv : div_rn(v[i][j], d);
    const uint32_t w0 = enc_e4m3x4_inrange<HW>(f[0], f[1], f[2], f[3]);
    const uint32_t w1 = enc_e4m3x4_inrange<HW>(f[4], f[5], f[6], f[7]);
    if (a.q) {
      const int64_t r = r0 + row + a.q_row_off, c = c0 + cc;
      const int64_t off = a.paired ? (r >> 1) * 2 * a.ld_q + (c >> 6) * 128 + (r & 1) * 64 + (c & 63)
                                   : r * a.ld_q + c;
      *reinterpret_cast<uint2*>(a.q + g * a.gs_q + off) = make_uint2(w0, w1);
    }
    tile[row][(cc >> 2)] = w0;
    tile[row][(cc >> 2) + 1] = w1;
  }
  if (a.q && tid == 0) a.s[g * a.gs_s + ((r0 + a.q_row_off) >> 7) * a.ld_s + (c0 >> 7)] = s;
  if (!a.qt) return;
  __syncthreads();
  // transposed payload: thread -> columns [4 cg, +4) x rows [16 rg, +16), 4 x 4
  // byte blocks transposed with v_perm_b32; the 8 lanes of one cg write a whole
  // 128-byte row of the transpose
  const int rg = tid & 7, cg = tid >> 3;
  uint32_t cw[4][4];   // [column][4-row word]
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int rb = 16 * rg + 4 * k;
    const uint32_t in[4] = {tile[rb][cg], tile[rb + 1][cg], tile[rb + 2][cg], tile[rb + 3][cg]};
    uint32_t out[4];
    transpose4x4_bytes(in, out);
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) cw[c4][k] = out[c4];
  }
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4)
    *reinterpret_cast<uint4*>(a.qt + g * a.gs_qt + (c0 + 4 * cg + c4) * a.ld_qt + a.qt_col_off + r0 + 16 * rg) =
        make_uint4(cw[c4][0], cw[c4][1], cw[c4][2], cw[c4][3]);
  if (tid == 0) a.st[g * a.gs_st + (c0 >> 7) * a.ld_st + ((r0 + a.qt_col_off) >> 7)] = s;
}

// Up to 4 jobs with one tile grid: blockIdx.z = job * groups + group.
struct WeightQuantBatch {
  WeightQuantArgs job[4];
  int64_t groups;
};

// A batch's blocks in one linear order (column tile fastest, then row tile,
// then job-major groups: the order of fm_quantize_weight_batch's grid), and the
// range [first, first + count) of them one launch runs.
struct WeightSide {
  WeightQuantBatch b;
  int64_t tiles_x, tiles_y;   // cols / 128, rows / 128 of every job
  int64_t total;              // tiles_x * tiles_y * groups * jobs
  int64_t first, count;
  int src_f32;
};

// Block `first + i` of the batch, by a whole 256-thread workgroup.
__device__ __forceinline__ void weight_side_block(const WeightSide& ws, int64_t i) {
  __shared__ float red[256];
  __shared__ uint32_t tile[128][65];
  // 32-bit decode (the host keeps total < 2^31): 64-bit divisions are long
  // emulated sequences, as costly as a tile's own arithmetic
  const uint32_t blk = uint32_t(ws.first + i), tx = uint32_t(ws.tiles_x), ty = uint32_t(ws.tiles_y);
  const uint32_t gr = uint32_t(ws.b.groups);
  const uint32_t yz = blk / tx, x = blk - yz * tx;
  const uint32_t z = yz / ty, y = yz - z * ty;
  const uint32_t j = z / gr, g = z - j * gr;
  if (ws.src_f32) weight_quant_tile<float>(ws.b.job[j], g, y, x, red, tile);
  else weight_quant_tile<uint16_t>(ws.b.job[j], g, y, x, red, tile);
}

// Host side (fm_quant.hip): validate 1-4 jobs as fm_quantize_weight_batch does
// and describe them (first = count = 0); run blocks [first, first + count) as
// a launch of their own.
int make_weight_side(const FmWeightJob* jobs, int n_jobs, WeightSide& ws, const char* what);
int launch_weight_side(const WeightSide& ws, int64_t first, int64_t count, hipStream_t s);

}  // namespace fm
