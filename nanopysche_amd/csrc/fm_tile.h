// 128x128 tile producer: one workgroup (256 threads, 4 wave64) turns a
// 128-row x 128-column tile of fp32 values -- produced on the fly by a source
// functor -- into
//   * a row-major output   (bf16, or e4m3 with 1x128 / 1x32 block scales), and/or
//   * a transposed output  (bf16, or e4m3 with 128x1 / 32x1 block scales),
// reading the source exactly once.  A source may yield NOUT values per
// element (SwiGLU backward yields dg and du), each with its own column offset
// in the outputs.  HBM-bound: 16-byte loads, 8-byte row stores (8 lanes cover
// one 64-byte half of a row block), 16-byte transposed stores.
//
// LDS staging for the transposed output:
//   QK_POW2  -- per output, e4m3 codes [128][128 + 4 pad] + one row scale per
//               row (17 KiB): the transposed output is the scaling-aware
//               transpose of the row output, so the codes are all it needs
//               (pow2_tile).
//   QK_BLOCK -- e4m3 codes already in the column scale (17 KiB); the values
//               stay in registers (block_tile).
//   others   -- fp32 values [128][129] (66 KiB), one output at a time.
// A launch without the transposed output uses no LDS (rows_tile).
#pragma once

#include "fm_common.h"
#include "../../include/fm_hip.h"

// e4m3 / bf16 conversion: the gfx950 convert instructions, or the integer
// routines of fm_common.h.  Both are bit-identical (checked on the GPU by
// fm_convert_check); the hardware path is the default.
#ifndef FM_HW_CVT
#define FM_HW_CVT 1
#endif

namespace fm {

enum QuantKind : int {
  QK_BF16 = 0,   // no quantisation, bf16 payload
  QK_BLOCK = 1,  // e4m3, fp32 scale = amax/448 per 128 block
  QK_POW2 = 2,   // e4m3, power-of-two fp32 scale per 128 block; transposed
                 // output is the scaling-aware transpose of the row output
  QK_MX = 3,     // e4m3, e8m0 scale per 32 block (OCP MX)
};

struct TileOut {
  int kind;              // QuantKind (dispatched to a template argument)
  // row-major output (nullptr = not wanted)
  void* row_q;           // bf16 or e4m3 [rows, *] with pitch ld_row (elements)
  int64_t ld_row;
  void* row_s;           // fp32 per 128 block or e8m0 per 32 block of a row:
  int64_t rs_row, rs_kb; //   row_s[row * rs_row + block * rs_kb]
  // transposed output (nullptr = not wanted); requires rows % 128 == 0
  void* col_q;           // bf16 or e4m3 [*, rows] with pitch ld_col (elements)
  int64_t ld_col;
  void* col_s;           // fp32 [rows/128, *] or e8m0 [rows/32, *]; pitch ld_col_s
  int64_t ld_col_s;
  int64_t col_off[2];    // output column offset of source value 0 / 1
  const int32_t* tile_valid;  // optional: skip 128-row tile t when tile_valid[t] < 0
  int paired;            // e4m3 row output in the paired-row layout (FM_ROWS_PAIRED)
  int col_paired;        // e4m3 transposed output in the paired-row layout (FM_COLS_PAIRED)
};

constexpr int kTileLdsPitch = 129;

// ------------------------------------------------------------- conversions ----
template <bool HW>
__device__ __forceinline__ uint32_t enc_e4m3x4(float a, float b, float c, float d) {
  if constexpr (HW) {
    return hw_e4m3x4(clamp448_med3(a), clamp448_med3(b), clamp448_med3(c), clamp448_med3(d));
  } else {
    return uint32_t(f32_to_e4m3(clamp448(a))) | (uint32_t(f32_to_e4m3(clamp448(b))) << 8) |
           (uint32_t(f32_to_e4m3(clamp448(c))) << 16) | (uint32_t(f32_to_e4m3(clamp448(d))) << 24);
  }
}
template <bool HW>
__device__ __forceinline__ uint32_t enc_bf16x2(float a, float b) {
  if constexpr (HW) return hw_bf16x2(a, b);
  else return uint32_t(f32_to_bf16(a)) | (uint32_t(f32_to_bf16(b)) << 16);
}

// e4m3 of four values of magnitude at most 464, without a clamp: both
// conversions round to nearest-even and give NaN only above 464 (the OCP
// non-saturating rule), so such values encode as if clamped to +-448.  Block
// quantisers produce them: a power-of-two scale bounds |x / s| by 448 exactly,
// an fp32 scale RN(amax / 448) by 448 (1 + 2^-24) before rounding.  MX scales
// (e8m0 from the amax exponent) allow up to 512 and keep the clamp.
template <bool HW>
__device__ __forceinline__ uint32_t enc_e4m3x4_inrange(float a, float b, float c, float d) {
  if constexpr (HW) {
    return hw_e4m3x4(a, b, c, d);
  } else {
    return uint32_t(f32_to_e4m3(a)) | (uint32_t(f32_to_e4m3(b)) << 8) | (uint32_t(f32_to_e4m3(c)) << 16) |
           (uint32_t(f32_to_e4m3(d)) << 24);
  }
}

// Lane exchanges for maxima of non-negative floats, done on their bit
// patterns (integer order equals float order for them, and integer max needs
// no NaN canonicalisation).  DPP within rows of 16 lanes: quad_perm [1,0,3,2],
// quad_perm [2,3,0,1], row_half_mirror (lane i <- 7 - i within 8), row_ror:8
// (lane i <- i ^ 8 within 16).
template <int CTRL>
__device__ __forceinline__ int dpp_move(int v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xf, 0xf, false);
}
constexpr int kDppQuadSwap1 = 0xb1, kDppQuadSwap2 = 0x4e, kDppRowHalfMirror = 0x141, kDppRowRor8 = 0x128;

// max over the 4 lanes of a quad
__device__ __forceinline__ float group_max4(float v) {
  int u = __builtin_bit_cast(int, v);
  u = max(u, dpp_move<kDppQuadSwap1>(u));
  u = max(u, dpp_move<kDppQuadSwap2>(u));
  return __builtin_bit_cast(float, u);
}
// max over 8 consecutive lanes (8-aligned): quad maxima, then the half mirror
// pairs quad 0 with quad 1
__device__ __forceinline__ float group_max8(float v) {
  int u = __builtin_bit_cast(int, group_max4(v));
  u = max(u, dpp_move<kDppRowHalfMirror>(u));
  return __builtin_bit_cast(float, u);
}
// max over the 8 lanes l, l ^ 8, l ^ 16, ..., l ^ 56 (same l % 8): row_ror:8,
// then v_permlane16_swap / v_permlane32_swap with both operands v, which
// leave {v[l], v[l ^ 16]} / {v[l], v[l ^ 32]} in their two results.
__device__ __forceinline__ float max_across_rowgroups(float v) {
  int u = __builtin_bit_cast(int, v);
  u = max(u, dpp_move<kDppRowRor8>(u));
  const auto a = __builtin_amdgcn_permlane16_swap(uint32_t(u), uint32_t(u), false, false);
  u = max(int(a[0]), int(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(uint32_t(u), uint32_t(u), false, false);
  u = max(int(b[0]), int(b[1]));
  return __builtin_bit_cast(float, u);
}

// 8 bf16 (one 16-byte load) -> 8 floats
__device__ __forceinline__ void unpack8_bf16(const uint4& pk, float v[8]) {
  const uint32_t q[4] = {pk.x, pk.y, pk.z, pk.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = u2f(q[i] << 16);
    v[2 * i + 1] = u2f(q[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint64_t pack8_e4m3(const uint8_t* b) {
  uint64_t r = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) r |= uint64_t(b[i]) << (8 * i);
  return r;
}

// Source functor contract:
//   static constexpr int kOut;                       // values per element (1 or 2)
//   struct Raw;                                      // what the loads of 8 columns return
//   __device__ Raw fetch(int64_t row, int64_t col) const;
//   __device__ void compute(const Raw& r, float v[kOut][8]) const;
// fetch issues the (branch-free) loads of columns [col, col+8) of logical row
// `row`; compute turns them into values (zeros for rows the source treats as
// padding).  The kernel fetches all of a thread's rows before computing any,
// so their loads overlap, and converts one row at a time.
//
// Thread layout: lane8 = tid % 8, row group rg = tid / 8 (0..31); a thread
// owns rows rg + 32 it (it = 0..3) and, in each, the two 8-column segments
// [64 h + 8 lane8, +8) (h = 0, 1).  One load instruction of a wave covers 8
// rows x 128 contiguous bytes of bf16 per row; the 8 lanes of a row group hold
// a whole 128-column block, so a row block's scale costs one 8-lane reduction
// per 16 values.
constexpr int kRowsPerThread = 4;

// Row-output addresses of one thread for one output: segment 0 of its row
// and the scale of that row block (MX: of segment 0's 32-column block);
// segment 1 is 64 columns (two MX blocks) further.  next() moves 32 rows down.
// In the paired-row layout (e4m3 only) row r's 64-column piece b sits at
// (r >> 1) * 2 ld + b * 128 + (r & 1) * 64, so segment 1 is 128 bytes on and
// 32 rows down is still 32 ld bytes on.
template <int KIND>
struct RowPtr {
  uintptr_t q, s;
  int64_t q_step, s_step, s_seg, q_seg;
  __device__ __forceinline__ RowPtr(const TileOut& o, int64_t row, int64_t ocol) {
    constexpr int64_t qb = KIND == QK_BF16 ? 2 : 1;
    const int64_t c = ocol + 8 * (threadIdx.x & 7);
    if (KIND != QK_BF16 && o.paired) {
      q = uintptr_t(o.row_q) + uintptr_t((row >> 1) * 2 * o.ld_row + (c >> 6) * 128 + (row & 1) * 64 + (c & 63));
      q_seg = 128;
    } else {
      q = uintptr_t(o.row_q) + uintptr_t((row * o.ld_row + c) * qb);
      q_seg = 64 * qb;
    }
    q_step = 32 * o.ld_row * qb;
    if (KIND == QK_MX) {
      s = uintptr_t(o.row_s) + uintptr_t(row * o.rs_row + (c >> 5) * o.rs_kb);
      s_step = 32 * o.rs_row;
      s_seg = 2 * o.rs_kb;
    } else {
      s = uintptr_t(o.row_s) + uintptr_t(4 * (row * o.rs_row + (ocol >> 7) * o.rs_kb));
      s_step = 128 * o.rs_row;
      s_seg = 0;
    }
  }
  __device__ __forceinline__ uintptr_t qseg(int h) const { return q + uintptr_t(h * q_seg); }
  __device__ __forceinline__ void next() {
    q += q_step;
    s += s_step;
  }
};

// Row output of one thread's 16 values of one row (v[h] = segment h): e4m3
// codes with the row block's scale (or bf16), stored when `store`; returns the
// code words {seg 0 cols 0-3, seg 0 cols 4-7, seg 1 cols 0-3, seg 1 cols 4-7}.
template <int KIND, bool HW>
__device__ __forceinline__ uint4 row_quant(const float (&v)[2][8], const RowPtr<KIND>& p, bool store, float& sc) {
  const int lane8 = threadIdx.x & 7;
  uint32_t w[4] = {0, 0, 0, 0};
  sc = 0.f;
  if constexpr (KIND == QK_BF16) {
    if (store) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
        st_global(reinterpret_cast<void*>(p.qseg(h)),
                  make_uint4(enc_bf16x2<HW>(v[h][0], v[h][1]), enc_bf16x2<HW>(v[h][2], v[h][3]),
                             enc_bf16x2<HW>(v[h][4], v[h][5]), enc_bf16x2<HW>(v[h][6], v[h][7])));
    }
    return make_uint4(0, 0, 0, 0);
  } else if constexpr (KIND == QK_MX) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float am = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(v[h][i]));
      const uint32_t code = mx_code(group_max4(am));
      const float inv = mx_inv_scale(code);
      w[2 * h] = enc_e4m3x4<HW>(v[h][0] * inv, v[h][1] * inv, v[h][2] * inv, v[h][3] * inv);
      w[2 * h + 1] = enc_e4m3x4<HW>(v[h][4] * inv, v[h][5] * inv, v[h][6] * inv, v[h][7] * inv);
      if (store && (lane8 & 3) == 0) st_global(reinterpret_cast<uint8_t*>(p.s + h * p.s_seg), uint8_t(code));
    }
  } else {
    float am = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(v[h][i]));
    sc = block_scale_dev(group_max8(am), KIND == QK_POW2);
    if constexpr (KIND == QK_POW2) {
      const float inv = pow2_recip(sc);  // exact: sc is a power of two, |v * inv| <= 448
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        w[2 * h] = enc_e4m3x4_inrange<HW>(v[h][0] * inv, v[h][1] * inv, v[h][2] * inv, v[h][3] * inv);
        w[2 * h + 1] = enc_e4m3x4_inrange<HW>(v[h][4] * inv, v[h][5] * inv, v[h][6] * inv, v[h][7] * inv);
      }
    } else {
      const Recip d = recip_of(sc);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        w[2 * h] = enc_e4m3x4_inrange<HW>(div_rn(v[h][0], d), div_rn(v[h][1], d), div_rn(v[h][2], d),
                                          div_rn(v[h][3], d));
        w[2 * h + 1] = enc_e4m3x4_inrange<HW>(div_rn(v[h][4], d), div_rn(v[h][5], d), div_rn(v[h][6], d),
                                              div_rn(v[h][7], d));
      }
    }
    if (store && lane8 == 0) st_global(reinterpret_cast<float*>(p.s), sc);
  }
  if (store) {
    st_global(reinterpret_cast<void*>(p.qseg(0)), make_uint2(w[0], w[1]));
    st_global(reinterpret_cast<void*>(p.qseg(1)), make_uint2(w[2], w[3]));
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Fetch of a thread's rows rg + 32 it, both segments: rows past the end
// re-read the last row (a full tile takes the unclamped path, whose addresses
// are a base plus multiples of 32 rows).
template <class Src>
__device__ __forceinline__ void fetch_rows(const Src& src, typename Src::Raw (&raw)[kRowsPerThread][2],
                                           int64_t rows, int64_t row0, int64_t col0) {
  const int64_t r = row0 + (threadIdx.x >> 3);
  const int64_t c = col0 + 8 * (threadIdx.x & 7);
  if (row0 + 128 <= rows) {
#pragma unroll
    for (int it = 0; it < kRowsPerThread; ++it)
#pragma unroll
      for (int h = 0; h < 2; ++h) raw[it][h] = src.fetch(r + 32 * it, c + 64 * h);
  } else {
#pragma unroll
    for (int it = 0; it < kRowsPerThread; ++it) {
      const int64_t g = r + 32 * it < rows ? r + 32 * it : rows - 1;
#pragma unroll
      for (int h = 0; h < 2; ++h) raw[it][h] = src.fetch(g, c + 64 * h);
    }
  }
}

// Rows rg + 32 (it0 + k), k < N, of a full tile (no clamping): a batch of
// a thread's rows, for sources whose raw values of all four rows would hold
// too many registers.
template <int N, class Src>
__device__ __forceinline__ void fetch_row_batch(const Src& src, typename Src::Raw (&raw)[N][2], int64_t row0,
                                                int64_t col0, int it0) {
  const int64_t r = row0 + (threadIdx.x >> 3) + 32 * it0;
  const int64_t c = col0 + 8 * (threadIdx.x & 7);
#pragma unroll
  for (int k = 0; k < N; ++k)
#pragma unroll
    for (int h = 0; h < 2; ++h) raw[k][h] = src.fetch(r + 32 * k, c + 64 * h);
}

// Values of one row: v[oi][h][i] for output oi, segment h.
template <class Src>
__device__ __forceinline__ void compute_row(const Src& src, const typename Src::Raw (&raw)[2],
                                            float (&v)[Src::kOut][2][8]) {
  float t[2][Src::kOut][8];
  src.compute(raw[0], t[0]);
  src.compute(raw[1], t[1]);
#pragma unroll
  for (int oi = 0; oi < Src::kOut; ++oi)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) v[oi][h][i] = t[h][oi][i];
}

// 4x4 byte transpose: out[c] byte b = in[b] byte c.
__device__ __forceinline__ void transpose4x4_bytes(const uint32_t (&in)[4], uint32_t (&out)[4]) {
  const uint32_t lo01 = __builtin_amdgcn_perm(in[1], in[0], 0x05010400u);  // i0b0 i1b0 i0b1 i1b1
  const uint32_t hi01 = __builtin_amdgcn_perm(in[1], in[0], 0x07030602u);  // i0b2 i1b2 i0b3 i1b3
  const uint32_t lo23 = __builtin_amdgcn_perm(in[3], in[2], 0x05010400u);
  const uint32_t hi23 = __builtin_amdgcn_perm(in[3], in[2], 0x07030602u);
  out[0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
  out[1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
}

// Word index of columns [4 cw, 4 cw + 4) of row `row` in a [128][33]-word
// LDS code tile.  The transposed reader below has lanes (rg, cg) read rows
// 16 rg + j; XOR-ing the word column with 8 in rows 64..127 puts its 64 lanes
// on 64 distinct banks (gfx950 LDS: 64 banks of 4 bytes; rows 64 apart would
// otherwise share one).  Groups of 4 aligned words stay together.
__device__ __forceinline__ int code_idx(int row, int cw) { return row * 33 + (cw ^ (8 * ((row >> 6) & 1))); }

// Transposed store of a 128x128 e4m3 tile staged in LDS as code words
// (code[code_idx(row, c / 4)] holds columns [c, c+4) of a row): thread -> columns
// [4 cg, +4) x rows [16 rg, +16); the 8 lanes of one cg write a whole
// 128-byte row of the transpose.  `tx` maps the four codes of one word (one
// row, four columns) to their values in the transposed output; the identity
// when the codes are already in the column scale.
// `paired`: the transposed output in the paired-row layout (its rows -- the
// source columns -- 2p and 2p + 1 interleaved in 64-byte pieces).
template <class TX>
__device__ __forceinline__ void store_transposed_codes(const uint32_t* code, uint8_t* qt8, int64_t ld_col,
                                                       int64_t ocol, int64_t row0, TX tx, bool paired = false) {
  const int tid = threadIdx.x;
  const int rg = tid & 7, cg = tid >> 3;
  uint32_t w[4][4];  // [column][4-row word]
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t in[4], out[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int row = 16 * rg + 4 * k + b;
      in[b] = tx(code[code_idx(row, cg)], row);
    }
    transpose4x4_bytes(in, out);
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) w[c4][k] = out[c4];
  }
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4) {
    const int64_t f = ocol + 4 * cg + c4, t = row0 + 16 * rg;
    const int64_t off = paired ? (f >> 1) * 2 * ld_col + (t >> 6) * 128 + (f & 1) * 64 + (t & 63) : f * ld_col + t;
    *reinterpret_cast<uint4*>(qt8 + off) = make_uint4(w[c4][0], w[c4][1], w[c4][2], w[c4][3]);
  }
}

// LDS word index of segment h of row r (this thread's two words) in a code tile
__device__ __forceinline__ int code_word(int r, int h) { return code_idx(r, 16 * h + 2 * (threadIdx.x & 7)); }

// Row output only: each row is quantised as soon as it is computed; no LDS.
template <class Src, int KIND, bool HW>
__device__ __forceinline__ void rows_tile(const Src& src, const TileOut& o, int64_t rows, int64_t row0,
                                          int64_t col0) {
  constexpr int NOUT = Src::kOut;
  typename Src::Raw raw[kRowsPerThread][2];
  fetch_rows(src, raw, rows, row0, col0);
  const int64_t r = row0 + (threadIdx.x >> 3);
  RowPtr<KIND> p[2] = {RowPtr<KIND>(o, r, col0 + o.col_off[0]), RowPtr<KIND>(o, r, col0 + o.col_off[NOUT - 1])};
#pragma unroll
  for (int it = 0; it < kRowsPerThread; ++it) {
    float v[NOUT][2][8];
    compute_row(src, raw[it], v);
    const bool ok = r + 32 * it < rows;
#pragma unroll
    for (int oi = 0; oi < NOUT; ++oi) {
      float sc;
      row_quant<KIND, HW>(v[oi], p[oi], ok, sc);
      p[oi].next();
    }
  }
}

// Power-of-two recipe with the transposed output: both outputs of a
// two-output source are quantised as soon as a row is computed (the
// transposed output is the scaling-aware transpose of the row output, so the
// e4m3 codes + row scales in LDS are all it needs, 17 KiB per output); no row
// values stay in registers.
template <class Src, bool HW>
__device__ __forceinline__ void pow2_tile(const Src& src, const TileOut& o, int64_t rows, int64_t row0,
                                          int64_t col0, bool want_row) {
  constexpr int NOUT = Src::kOut;
  const int tid = threadIdx.x;
  __shared__ float p_red[NOUT];
  __shared__ float p_rscale[NOUT][128];
  __shared__ __attribute__((aligned(16))) uint32_t p_code[NOUT][128 * 33];
  // A two-output source fetches its rows in two batches of two: the raw
  // values of four rows would keep the kernel at two waves per SIMD.
  constexpr int kBatch = NOUT == 2 ? 2 : kRowsPerThread;
  typename Src::Raw raw[kBatch][2];
  const int64_t rg = tid >> 3;
  RowPtr<QK_POW2> p[2] = {RowPtr<QK_POW2>(o, row0 + rg, col0 + o.col_off[0]),
                          RowPtr<QK_POW2>(o, row0 + rg, col0 + o.col_off[NOUT - 1])};
#pragma unroll
  for (int it = 0; it < kRowsPerThread; ++it) {
    // rows % 128 == 0: every row is in range
    if (it % kBatch == 0) fetch_row_batch<kBatch>(src, raw, row0, col0, it);
    float v[NOUT][2][8];
    compute_row(src, raw[it % kBatch], v);
    const int r = int(rg) + 32 * it;
#pragma unroll
    for (int oi = 0; oi < NOUT; ++oi) {
      float sc;
      const uint4 w = row_quant<QK_POW2, HW>(v[oi], p[oi], want_row, sc);
      p[oi].next();
      *reinterpret_cast<uint2*>(&p_code[oi][code_word(r, 0)]) = make_uint2(w.x, w.y);
      *reinterpret_cast<uint2*>(&p_code[oi][code_word(r, 1)]) = make_uint2(w.z, w.w);
      if ((tid & 7) == 0) p_rscale[oi][r] = sc;
    }
  }
  __syncthreads();
  // column scale of each output: the largest row scale of the tile
  if (tid < 64) {
#pragma unroll
    for (int oi = 0; oi < NOUT; ++oi) {
      float m = fmaxf(p_rscale[oi][tid], p_rscale[oi][tid + 64]);
      for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
      if (tid == 0) p_red[oi] = m;
    }
  }
  __syncthreads();
  // decode(q) * (s_row / s_col) is exact (powers of two) and at most 448.
  const int cg = tid >> 3;
#pragma unroll
  for (int oi = 0; oi < NOUT; ++oi) {
    const int64_t ocol = col0 + o.col_off[oi];
    const float st = p_red[oi];
    const float inv = pow2_recip(st);
    const float* rs = p_rscale[oi];
    store_transposed_codes(p_code[oi], static_cast<uint8_t*>(o.col_q), o.ld_col, ocol, row0,
                           [&](uint32_t word, int row) {
                             const float ratio = rs[row] * inv;
                             float d[4];
                             if constexpr (HW) {
                               hw_dec_e4m3x4(word, d);
                             } else {
#pragma unroll
                               for (int c4 = 0; c4 < 4; ++c4) d[c4] = e4m3_to_f32(uint8_t(word >> (8 * c4)));
                             }
                             return enc_e4m3x4_inrange<HW>(d[0] * ratio, d[1] * ratio, d[2] * ratio,
                                                           d[3] * ratio);
                           },
                           o.col_paired != 0);
    if ((tid & 7) == 0) {
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4)
        static_cast<float*>(o.col_s)[(row0 >> 7) * o.ld_col_s + ocol + 4 * cg + c4] = st;
    }
  }
}

// fp32 scale (amax / 448) with the 128x1 transposed output: the tile's values
// stay in registers; column amaxes are reduced across the 8 row groups of a
// wave by lane exchanges and across the 4 waves through LDS, each thread
// quantises its own values with their column's scale, and only the e4m3 codes
// pass through LDS (17 KiB).
template <class Src, bool HW>
__device__ __forceinline__ void block_tile(const Src& src, const TileOut& o, int64_t rows, int64_t row0,
                                           int64_t col0, bool want_row) {
  constexpr int NOUT = Src::kOut;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane8 = tid & 7;
  __shared__ __attribute__((aligned(16))) float b_red[4][128];
  __shared__ __attribute__((aligned(16))) float b_sd[128];
  __shared__ __attribute__((aligned(16))) float b_ny[128];
  __shared__ __attribute__((aligned(16))) uint32_t b_code[128 * 33];
  float vv[kRowsPerThread][NOUT][2][8];
  {
    typename Src::Raw raw[kRowsPerThread][2];
    fetch_rows(src, raw, rows, row0, col0);
#pragma unroll
    for (int it = 0; it < kRowsPerThread; ++it) compute_row(src, raw[it], vv[it]);
  }
  const int rg = tid >> 3;
#pragma unroll
  for (int oi = 0; oi < NOUT; ++oi) {
    const int64_t ocol = col0 + o.col_off[oi];
    float cm[2][8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) cm[h][i] = 0.f;
    RowPtr<QK_BLOCK> p(o, row0 + rg, ocol);
#pragma unroll
    for (int it = 0; it < kRowsPerThread; ++it) {
      float sc;
      row_quant<QK_BLOCK, HW>(vv[it][oi], p, want_row, sc);
      p.next();
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 8; ++i) cm[h][i] = fmaxf(cm[h][i], fabsf(vv[it][oi][h][i]));
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) cm[h][i] = max_across_rowgroups(cm[h][i]);
    if (oi > 0) __syncthreads();  // the previous output's transposed reads are done
    if ((tid & 63) < 8) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float* dst = &b_red[wave][64 * h + 8 * lane8];
        *reinterpret_cast<float4*>(dst) = make_float4(cm[h][0], cm[h][1], cm[h][2], cm[h][3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(cm[h][4], cm[h][5], cm[h][6], cm[h][7]);
      }
    }
    __syncthreads();
    if (tid < 128) {
      const float m = fmaxf(fmaxf(b_red[0][tid], b_red[1][tid]), fmaxf(b_red[2][tid], b_red[3][tid]));
      const float s = block_scale_dev(m, false);
      const Recip d = recip_of(s);
      b_sd[tid] = d.sd;
      b_ny[tid] = d.ny;
      static_cast<float*>(o.col_s)[(row0 >> 7) * o.ld_col_s + ocol + tid] = s;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 64 * h + 8 * lane8;
      const float4 s0 = *reinterpret_cast<const float4*>(&b_sd[c]);
      const float4 s1 = *reinterpret_cast<const float4*>(&b_sd[c + 4]);
      const float4 y0 = *reinterpret_cast<const float4*>(&b_ny[c]);
      const float4 y1 = *reinterpret_cast<const float4*>(&b_ny[c + 4]);
      const Recip d[8] = {{s0.x, y0.x}, {s0.y, y0.y}, {s0.z, y0.z}, {s0.w, y0.w},
                          {s1.x, y1.x}, {s1.y, y1.y}, {s1.z, y1.z}, {s1.w, y1.w}};
#pragma unroll
      for (int it = 0; it < kRowsPerThread; ++it) {
        const float* v = vv[it][oi][h];
        const uint32_t w0 = enc_e4m3x4_inrange<HW>(div_rn(v[0], d[0]), div_rn(v[1], d[1]), div_rn(v[2], d[2]),
                                                   div_rn(v[3], d[3]));
        const uint32_t w1 = enc_e4m3x4_inrange<HW>(div_rn(v[4], d[4]), div_rn(v[5], d[5]), div_rn(v[6], d[6]),
                                                   div_rn(v[7], d[7]));
        *reinterpret_cast<uint2*>(&b_code[code_word(rg + 32 * it, h)]) = make_uint2(w0, w1);
      }
    }
    __syncthreads();
    store_transposed_codes(b_code, static_cast<uint8_t*>(o.col_q), o.ld_col, ocol, row0,
                           [](uint32_t word, int) { return word; }, o.col_paired != 0);
  }
}

// MX (32x1) with the transposed output.  Rows are dealt so that wave w holds
// the tile's 32-row block w: thread (w, lane) owns rows 32 w + 8 it +
// lane / 8 (it = 0..3), in each the two 8-column segments of the other
// layouts, so one row-store instruction covers 8 consecutive rows (whole
// 128-byte lines of the paired-row layout, whose rows 2p and 2p + 1 share
// them; with 4 consecutive rows per thread each line took two stores).  A
// block's column amax is then the maximum over the thread's own 4 rows and
// the wave's 8 row groups (lane exchanges): the scales need no LDS and no
// barrier.  Each row's values stay in registers until the column scales are
// known (4 rows x 16 columns per output), each thread encodes them, and only
// the e4m3 codes pass through LDS (16.5 KiB per output) for the transposed
// stores -- one barrier per tile.  Values, scales and encodes are those of the
// row blocks and of staging the fp32 tile in LDS, so the bytes are the same.
template <class Src, bool HW>
__device__ __forceinline__ void mx_tile(const Src& src, const TileOut& o, int64_t rows, int64_t row0,
                                        int64_t col0, bool want_row) {
  constexpr int NOUT = Src::kOut;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, lane8 = tid & 7;
  __shared__ __attribute__((aligned(16))) uint32_t m_code[NOUT][128 * 33];
  const int rb = 32 * wave + (lane >> 3);   // the thread's row it is rb + 8 it
  typename Src::Raw raw[kRowsPerThread][2];
  {
    const int64_t c = col0 + 8 * lane8;   // rows % 128 == 0: every row is in range
#pragma unroll
    for (int it = 0; it < kRowsPerThread; ++it)
#pragma unroll
      for (int h = 0; h < 2; ++h) raw[it][h] = src.fetch(row0 + rb + 8 * it, c + 64 * h);
  }
  float v[kRowsPerThread][NOUT][2][8];
  float cm[NOUT][2][8];
#pragma unroll
  for (int it = 0; it < kRowsPerThread; ++it) {
    compute_row(src, raw[it], v[it]);
#pragma unroll
    for (int oi = 0; oi < NOUT; ++oi) {
      const RowPtr<QK_MX> p(o, row0 + rb + 8 * it, col0 + o.col_off[oi]);
      float sc;
      row_quant<QK_MX, HW>(v[it][oi], p, want_row, sc);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          cm[oi][h][i] = it == 0 ? fabsf(v[it][oi][h][i]) : fmaxf(cm[oi][h][i], fabsf(v[it][oi][h][i]));
    }
  }
  uint8_t* const cs = static_cast<uint8_t*>(o.col_s) + ((row0 + 32 * wave) >> 5) * o.ld_col_s + col0;
#pragma unroll
  for (int oi = 0; oi < NOUT; ++oi)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t code[8];
      float inv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        code[i] = mx_code(max_across_rowgroups(cm[oi][h][i]));
        inv[i] = mx_inv_scale(code[i]);
      }
      if (lane < 8) {   // the 8 scale bytes of this lane's columns (one 8-byte store when aligned)
        uint8_t* d = cs + o.col_off[oi] + 64 * h + 8 * lane8;
        if ((reinterpret_cast<uintptr_t>(d) & 7) == 0) {
          *reinterpret_cast<uint2*>(d) = make_uint2(code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24),
                                                    code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24));
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) d[i] = uint8_t(code[i]);
        }
      }
#pragma unroll
      for (int it = 0; it < kRowsPerThread; ++it) {
        const float* x = v[it][oi][h];
        const uint32_t w0 = enc_e4m3x4<HW>(x[0] * inv[0], x[1] * inv[1], x[2] * inv[2], x[3] * inv[3]);
        const uint32_t w1 = enc_e4m3x4<HW>(x[4] * inv[4], x[5] * inv[5], x[6] * inv[6], x[7] * inv[7]);
        *reinterpret_cast<uint2*>(&m_code[oi][code_word(rb + 8 * it, h)]) = make_uint2(w0, w1);
      }
    }
  __syncthreads();
#pragma unroll
  for (int oi = 0; oi < NOUT; ++oi)
    store_transposed_codes(m_code[oi], static_cast<uint8_t*>(o.col_q), o.ld_col, col0 + o.col_off[oi], row0,
                           [](uint32_t word, int) { return word; }, o.col_paired != 0);
}

// bf16 transposed outputs: fp32 values staged in LDS [128][129] (66 KiB),
// one output at a time.
template <class Src, int KIND, bool HW>
__device__ __forceinline__ void staged_tile(const Src& src, const TileOut& o, int64_t rows, int64_t row0,
                                            int64_t col0, bool want_row) {
  constexpr int NOUT = Src::kOut;
  const int tid = threadIdx.x;
  float vv[kRowsPerThread][NOUT][2][8];
  {
    typename Src::Raw raw[kRowsPerThread][2];
    fetch_rows(src, raw, rows, row0, col0);
#pragma unroll
    for (int it = 0; it < kRowsPerThread; ++it) compute_row(src, raw[it], vv[it]);
  }
  __shared__ float lds_val[128 * kTileLdsPitch];
  const int rg = tid >> 3, lane8 = tid & 7;
#pragma unroll
  for (int oi = 0; oi < NOUT; ++oi) {
    const int64_t ocol = col0 + o.col_off[oi];  // output column of this tile
    RowPtr<KIND> p(o, row0 + rg, ocol);
#pragma unroll
    for (int it = 0; it < kRowsPerThread; ++it) {
      const int r = rg + 32 * it;
      float sc;
      row_quant<KIND, HW>(vv[it][oi], p, want_row, sc);
      p.next();
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 8; ++i) lds_val[r * kTileLdsPitch + 64 * h + 8 * lane8 + i] = vv[it][oi][h][i];
    }
    __syncthreads();

    // thread -> column c = tid % 128, rows [64*h, 64*h + 64)
    const int c = tid & 127, h = tid >> 7;
    const int64_t gcol = ocol + c;
    if constexpr (KIND == QK_MX) {
      uint8_t* qt8 = static_cast<uint8_t*>(o.col_q);
      for (int b = 0; b < 2; ++b) {  // two 32-row MX blocks per thread
        const int rb = 64 * h + 32 * b;
        float m = 0.f;
        for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(lds_val[(rb + i) * kTileLdsPitch + c]));
        const uint32_t code = mx_code(m);
        const float inv = mx_inv_scale(code);
        for (int r16 = 0; r16 < 32; r16 += 16) {
          uint32_t w[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const float* pv = &lds_val[(rb + r16 + 4 * k) * kTileLdsPitch + c];
            w[k] = enc_e4m3x4<HW>(pv[0] * inv, pv[kTileLdsPitch] * inv, pv[2 * kTileLdsPitch] * inv,
                                  pv[3 * kTileLdsPitch] * inv);
          }
          *reinterpret_cast<uint4*>(qt8 + gcol * o.ld_col + row0 + rb + r16) = make_uint4(w[0], w[1], w[2], w[3]);
        }
        static_cast<uint8_t*>(o.col_s)[((row0 + rb) >> 5) * o.ld_col_s + gcol] = uint8_t(code);
      }
    } else {  // bf16 transpose
      uint16_t* qt16 = static_cast<uint16_t*>(o.col_q);
      for (int r8 = 0; r8 < 64; r8 += 8) {
        const float* pv = &lds_val[(64 * h + r8) * kTileLdsPitch + c];
        const uint4 pk = make_uint4(enc_bf16x2<HW>(pv[0], pv[kTileLdsPitch]),
                                    enc_bf16x2<HW>(pv[2 * kTileLdsPitch], pv[3 * kTileLdsPitch]),
                                    enc_bf16x2<HW>(pv[4 * kTileLdsPitch], pv[5 * kTileLdsPitch]),
                                    enc_bf16x2<HW>(pv[6 * kTileLdsPitch], pv[7 * kTileLdsPitch]));
        *reinterpret_cast<uint4*>(qt16 + gcol * o.ld_col + row0 + 64 * h + r8) = pk;
      }
    }
    if (oi + 1 < NOUT) __syncthreads();  // LDS is reused by the next output
  }
}

// Per-tile view of a source: a source whose row -> address map is cheaper to
// resolve once per 128-row tile overloads this (found by argument-dependent
// lookup where the tile producer is instantiated).
template <class Src>
__device__ __forceinline__ Src tile_source(const Src& src, int64_t) {
  return src;
}

// One 128x128 tile at (row0, col0).
template <class Src, int KIND, bool HW, bool COL>
__device__ __forceinline__ void one_tile(const Src& src_all, const TileOut& o, int64_t rows, int64_t row0,
                                         int64_t col0) {
  const Src src = tile_source(src_all, row0);
  if constexpr (!COL) {
    rows_tile<Src, KIND, HW>(src, o, rows, row0, col0);
  } else {
    // the transposed output requires rows % 128 == 0: every row is in range
    const bool want_row = o.row_q != nullptr;
    if constexpr (KIND == QK_POW2) pow2_tile<Src, HW>(src, o, rows, row0, col0, want_row);
    else if constexpr (KIND == QK_BLOCK) block_tile<Src, HW>(src, o, rows, row0, col0, want_row);
    else if constexpr (KIND == QK_MX) mx_tile<Src, HW>(src, o, rows, row0, col0, want_row);
    else staged_tile<Src, KIND, HW>(src, o, rows, row0, col0, want_row);
  }
}

// COL: the transposed output is wanted (a separate instantiation, so a
// row-only launch allocates no LDS).  One workgroup per 128x128 tile; WALK:
// a grid capped below the row tiles (the launcher does so when tile_valid is
// given -- the rows of a local expert share are sized for every slot, and
// most of its tiles are then usually empty), where workgroup (x, y) takes
// the valid tiles among row tiles y, y + gridDim.y, ...  The validity of 64 such
// candidates comes from one load per lane and a ballot (the same in every
// wave), so an empty tile costs neither a workgroup launch nor a round trip
// of its own.
template <class Src, int KIND, bool COL, bool WALK>
__global__ __launch_bounds__(256) void tile_producer_kernel(Src src_all, TileOut o, int64_t rows) {
  constexpr bool HW = FM_HW_CVT != 0;
  const int64_t col0 = int64_t(blockIdx.x) * 128;
  if constexpr (!WALK) {
    if (o.tile_valid != nullptr && o.tile_valid[blockIdx.y] < 0) return;
    one_tile<Src, KIND, HW, COL>(src_all, o, rows, int64_t(blockIdx.y) * 128, col0);
  } else {
    const int64_t ntiles = (rows + 127) / 128;
    const int lane = threadIdx.x & 63;
    bool busy = false;
    for (int64_t base = blockIdx.y; base < ntiles; base += 64 * int64_t(gridDim.y)) {
      const int64_t cand = base + int64_t(lane) * gridDim.y;
      const bool ok = cand < ntiles && (o.tile_valid == nullptr || o.tile_valid[cand] >= 0);
      for (uint64_t m = __ballot(ok); m != 0; m &= m - 1) {
        if (busy) __syncthreads();   // the previous tile's LDS reads are done
        busy = true;
        one_tile<Src, KIND, HW, COL>(src_all, o, rows, (base + int64_t(__builtin_ctzll(m)) * gridDim.y) * 128,
                                     col0);
      }
    }
  }
}

// Validates a TileOut against the tile geometry; returns nonzero (with the
// error set) on a mismatch.  `cols` is the source's column count per output.
// TileOut from the C-ABI arguments; `kind` may carry FM_SCALES_KMAJOR.
inline TileOut make_tile_out(int kind, void* q, int64_t ld_q, void* s, int64_t ld_s, void* qt,
                             int64_t ld_qt, void* st, int64_t ld_st, int64_t off0, int64_t off1,
                             const int32_t* tile_valid) {
  const bool kmajor = (kind & FM_SCALES_KMAJOR) != 0;
  TileOut o{kind & ~(FM_SCALES_KMAJOR | FM_ROWS_PAIRED | FM_COLS_PAIRED), q, ld_q, s, kmajor ? 1 : ld_s,
            kmajor ? ld_s : 1, qt, ld_qt, st, ld_st, {off0, off1}, tile_valid, (kind & FM_ROWS_PAIRED) != 0,
            (kind & FM_COLS_PAIRED) != 0};
  return o;
}

inline int check_tile_out(const TileOut& o, int64_t rows, int64_t cols, int nout) {
  FM_REQUIRE(cols > 0 && cols % 128 == 0, "cols must be a positive multiple of 128 (got %lld)",
             (long long)cols);
  FM_REQUIRE(rows >= 0, "rows must be >= 0");
  FM_REQUIRE(o.kind >= QK_BF16 && o.kind <= QK_MX, "unknown quant kind %d", o.kind);
  FM_REQUIRE(o.row_q != nullptr || o.col_q != nullptr, "no output requested");
  const int64_t span = o.col_off[nout - 1] + cols;  // output columns touched
  FM_REQUIRE(o.col_off[0] % 128 == 0 && o.col_off[nout - 1] % 128 == 0, "column offsets must be multiples of 128");
  if (o.row_q != nullptr) {
    FM_REQUIRE(o.ld_row >= span, "row output pitch %lld < columns %lld", (long long)o.ld_row,
               (long long)span);
    FM_REQUIRE(o.ld_row % 8 == 0, "row output pitch must be a multiple of 8");
    FM_REQUIRE(!o.paired || (o.kind != QK_BF16 && o.ld_row % 64 == 0 && rows % 2 == 0),
               "paired rows need an e4m3 kind, a row pitch that is a multiple of 64 and an even row count");
    if (o.kind != QK_BF16) {
      FM_REQUIRE(o.row_s != nullptr, "row scale output missing");
      const int64_t nblk = o.kind == QK_MX ? span / 32 : span / 128;
      FM_REQUIRE((o.rs_kb == 1 && o.rs_row >= nblk) || (o.rs_row == 1 && o.rs_kb >= rows),
                 "row scale pitch too small");
    }
  }
  if (o.col_q != nullptr) {
    FM_REQUIRE(rows % 128 == 0, "transposed output needs rows %% 128 == 0 (got %lld)",
               (long long)rows);
    FM_REQUIRE(o.ld_col >= rows, "transposed output pitch too small");
    FM_REQUIRE(o.ld_col % 16 == 0, "transposed output pitch must be a multiple of 16");
    FM_REQUIRE(!o.col_paired || (o.kind != QK_BF16 && o.ld_col % 64 == 0),
               "paired transposed rows need an e4m3 kind and a pitch that is a multiple of 64");
    if (o.kind != QK_BF16) {
      FM_REQUIRE(o.col_s != nullptr, "transposed scale output missing");
      FM_REQUIRE(o.ld_col_s >= span, "transposed scale pitch too small");
    }
  }
  return 0;
}

template <class Src>
int launch_tile_producer(const Src& src, const TileOut& o, int64_t rows, int64_t cols,
                         hipStream_t stream, const char* what) {
  if (int rc = check_tile_out(o, rows, cols, Src::kOut)) return rc;
  if (rows == 0) return 0;
  // A capped grid keeps about kTileGridCap workgroups, 128 per CU: taken
  // when tile_valid is given and the tiles outnumber that (33,000 rows of
  // 14,336 columns, 264 x 112 tiles, stay at one tile per workgroup), or when
  // the row tiles exceed the grid's y limit.
  constexpr int64_t kTileGridCap = 32768;
  const int64_t gx = cols / 128, ntiles = (rows + 127) / 128;
  const int64_t cap = (kTileGridCap + gx - 1) / gx;
  const bool walk = cap < ntiles && (o.tile_valid != nullptr || ntiles > 65535);
  const dim3 grid{unsigned(gx), unsigned(walk ? cap : ntiles), 1u};
  const bool col = o.col_q != nullptr;
#define FM_TILE_LAUNCH2(K, C)                                                                                 \
  if (walk) hipLaunchKernelGGL((tile_producer_kernel<Src, K, C, true>), grid, dim3(256), 0, stream, src, o, rows); \
  else hipLaunchKernelGGL((tile_producer_kernel<Src, K, C, false>), grid, dim3(256), 0, stream, src, o, rows);
#define FM_TILE_LAUNCH(K)      \
  if (col) {                   \
    FM_TILE_LAUNCH2(K, true)   \
  } else {                     \
    FM_TILE_LAUNCH2(K, false)  \
  }
  switch (o.kind) {
    case QK_BF16: FM_TILE_LAUNCH(QK_BF16) break;
    case QK_BLOCK: FM_TILE_LAUNCH(QK_BLOCK) break;
    case QK_POW2: FM_TILE_LAUNCH(QK_POW2) break;
    default: FM_TILE_LAUNCH(QK_MX) break;
  }
#undef FM_TILE_LAUNCH2
#undef FM_TILE_LAUNCH
  return check_launch(what);
}

}  // namespace fm
