// 128x128 tile producer: one workgroup (256 threads, 4 wave64) turns a
// 128-row x 128-column tile of fp32 values -- produced on the fly by a source
// functor -- into
//   * a row-major output   (bf16, or e4m3 with 1x128 / 1x32 block scales), and/or
//   * a transposed output  (bf16, or e4m3 with 128x1 / 32x1 block scales),
// reading the source exactly once.  A source may yield NOUT values per
// element (SwiGLU backward yields dg and du), each with its own column offset
// in the outputs.  HBM-bound: 16-byte loads, 8-byte row stores (16 lanes cover
// one 128-byte row segment), 16-byte transposed stores.
//
// LDS staging for the transposed output:
//   QK_POW2  -- per output, e4m3 codes [128][128 + 4 pad] + one row scale per
//               row (17 KiB): the transposed output is the scaling-aware
//               transpose of the row output, so the codes are all it needs
//               (pow2_tile).
//   others   -- fp32 values [128][129] (66 KiB), one output at a time.
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

__device__ __forceinline__ float group_max16(float v) {
  // max over the 16 consecutive lanes that share a 128-column row block
  v = fmaxf(v, __shfl_xor(v, 1, 16));
  v = fmaxf(v, __shfl_xor(v, 2, 16));
  v = fmaxf(v, __shfl_xor(v, 4, 16));
  v = fmaxf(v, __shfl_xor(v, 8, 16));
  return v;
}
__device__ __forceinline__ float group_max4(float v) {
  v = fmaxf(v, __shfl_xor(v, 1, 4));
  v = fmaxf(v, __shfl_xor(v, 2, 4));
  return v;
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
//   struct Raw;                                      // what the loads of one row return
//   __device__ Raw fetch(int64_t row, int64_t col) const;
//   __device__ void compute(const Raw& r, float v[kOut][8]) const;
// fetch issues the (branch-free) loads of columns [col, col+8) of logical row
// `row`; compute turns them into values (zeros for rows the source treats as
// padding).  The kernel fetches all of a thread's rows before computing any,
// so their loads overlap, and converts one row at a time.
// Power-of-two recipe: both outputs of a two-output source are quantised as
// soon as a row is computed (the transposed output is the scaling-aware
// transpose of the row output, so e4m3 codes + row scales in LDS are all it
// needs, 17 KiB per output); no row values stay in registers.
template <class Src, bool HW>
__device__ __forceinline__ void pow2_tile(const Src& src, const TileOut& o, int64_t rows, int64_t row0,
                                          int64_t col0, int cpos, bool want_row, bool want_col) {
  constexpr int NOUT = Src::kOut;
  const int tid = threadIdx.x;
  __shared__ float p_red[NOUT];
  __shared__ float p_rscale[NOUT][128];
  __shared__ __attribute__((aligned(16))) uint32_t p_code[NOUT][128 * 33];
  typename Src::Raw raw[8];
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int64_t grow = row0 + (tid >> 4) + 16 * it;
    raw[it] = src.fetch(grow < rows ? grow : rows - 1, col0 + cpos);
  }
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    float v[NOUT][8];
    src.compute(raw[it], v);
    const int r = (tid >> 4) + 16 * it;
    const int64_t grow = row0 + r;
    const bool ok = grow < rows;
#pragma unroll
    for (int oi = 0; oi < NOUT; ++oi) {
      float am = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v[oi][i] = ok ? v[oi][i] : 0.f;
        am = fmaxf(am, fabsf(v[oi][i]));
      }
      const float sc = block_scale(group_max16(am), true);
      const float inv = 1.0f / sc;  // exact: sc is a power of two
      const uint32_t w0 = enc_e4m3x4<HW>(v[oi][0] * inv, v[oi][1] * inv, v[oi][2] * inv, v[oi][3] * inv);
      const uint32_t w1 = enc_e4m3x4<HW>(v[oi][4] * inv, v[oi][5] * inv, v[oi][6] * inv, v[oi][7] * inv);
      const int64_t ocol = col0 + o.col_off[oi];
      if (want_row && ok) {
        *reinterpret_cast<uint2*>(static_cast<uint8_t*>(o.row_q) + grow * o.ld_row + ocol + cpos) =
            make_uint2(w0, w1);
        if ((tid & 15) == 0) static_cast<float*>(o.row_s)[grow * o.rs_row + (ocol >> 7) * o.rs_kb] = sc;
      }
      if (want_col) {
        p_code[oi][r * 33 + (cpos >> 2)] = w0;
        p_code[oi][r * 33 + (cpos >> 2) + 1] = w1;
        if ((tid & 15) == 0) p_rscale[oi][r] = sc;
      }
    }
  }
  if (!want_col) return;
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
  // thread -> columns [4 cg, +4) (one LDS word per row) x rows [16 rg, +16):
  // the 8 lanes of one cg write a whole 128-byte row of the transpose.
  // decode(q) * (s_row / s_col) is exact (powers of two) and <= 448.
  uint8_t* qt8 = static_cast<uint8_t*>(o.col_q);
  const int rg = tid & 7, cg = tid >> 3;
#pragma unroll
  for (int oi = 0; oi < NOUT; ++oi) {
    const int64_t ocol = col0 + o.col_off[oi];
    const float st = p_red[oi];
    const float inv = 1.0f / st;  // exact: power of two
    uint32_t w[4][4];   // [column][4-row word]
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float f[4][4];    // [row][column]
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int row = 16 * rg + 4 * k + b;
        const float ratio = p_rscale[oi][row] * inv;
        const uint32_t word = p_code[oi][row * 33 + cg];
        float d[4];
        if constexpr (HW) {
          hw_dec_e4m3x4(word, d);
        } else {
#pragma unroll
          for (int c4 = 0; c4 < 4; ++c4) d[c4] = e4m3_to_f32(uint8_t(word >> (8 * c4)));
        }
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) f[b][c4] = d[c4] * ratio;
      }
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) w[c4][k] = enc_e4m3x4<HW>(f[0][c4], f[1][c4], f[2][c4], f[3][c4]);
    }
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4)
      *reinterpret_cast<uint4*>(qt8 + (ocol + 4 * cg + c4) * o.ld_col + row0 + 16 * rg) =
          make_uint4(w[c4][0], w[c4][1], w[c4][2], w[c4][3]);
    if (rg == 0) {
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4)
        static_cast<float*>(o.col_s)[(row0 >> 7) * o.ld_col_s + ocol + 4 * cg + c4] = st;
    }
  }
}

template <class Src, int KIND>
__global__ __launch_bounds__(256) void tile_producer_kernel(Src src, TileOut o, int64_t rows) {
  constexpr int NOUT = Src::kOut;
  constexpr bool HW = FM_HW_CVT != 0;
  const int64_t col0 = int64_t(blockIdx.x) * 128;
  const int64_t row0 = int64_t(blockIdx.y) * 128;
  if (o.tile_valid != nullptr && o.tile_valid[blockIdx.y] < 0) return;
  const int tid = threadIdx.x;
  const bool want_col = o.col_q != nullptr;
  const bool want_row = o.row_q != nullptr;

  // ---- phase 1: thread -> rows (tid/16) + 16*it, columns [8*(tid%16), +8).
  // All 8 rows are fetched before any is computed, so their loads are in
  // flight together; rows past the end re-read the last row and are zeroed by
  // a select.
  const int cpos = (tid & 15) * 8;
  if constexpr (KIND == QK_POW2) {
    pow2_tile<Src, HW>(src, o, rows, row0, col0, cpos, want_row, want_col);
    return;
  }
  float vv[8][NOUT][8];
  {
    typename Src::Raw raw[8];
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int64_t grow = row0 + (tid >> 4) + 16 * it;
      raw[it] = src.fetch(grow < rows ? grow : rows - 1, col0 + cpos);
    }
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      src.compute(raw[it], vv[it]);
      const bool ok = row0 + (tid >> 4) + 16 * it < rows;
#pragma unroll
      for (int q = 0; q < NOUT; ++q)
#pragma unroll
        for (int i = 0; i < 8; ++i) vv[it][q][i] = ok ? vv[it][q][i] : 0.f;
    }
  }

  // LDS for the transposed pass (one output at a time): fp32 values
  __shared__ float red[256];
  __shared__ float lds_val[128 * kTileLdsPitch];

#pragma unroll
  for (int oi = 0; oi < NOUT; ++oi) {
    const int64_t ocol = col0 + o.col_off[oi];  // output column of this tile
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int r = (tid >> 4) + 16 * it;
      const int64_t grow = row0 + r;
      const float* v = vv[it][oi];
      float am = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(v[i]));
      if (KIND == QK_BLOCK) {
        const float s = block_scale(group_max16(am), false);
        const float y = 1.0f / s;
        const uint32_t w0 = enc_e4m3x4<HW>(div_rn(v[0], s, y), div_rn(v[1], s, y), div_rn(v[2], s, y),
                                           div_rn(v[3], s, y));
        const uint32_t w1 = enc_e4m3x4<HW>(div_rn(v[4], s, y), div_rn(v[5], s, y), div_rn(v[6], s, y),
                                           div_rn(v[7], s, y));
        if (want_row && grow < rows) {
          *reinterpret_cast<uint2*>(static_cast<uint8_t*>(o.row_q) + grow * o.ld_row + ocol + cpos) =
              make_uint2(w0, w1);
          if ((tid & 15) == 0) static_cast<float*>(o.row_s)[grow * o.rs_row + (ocol >> 7) * o.rs_kb] = s;
        }
        if (want_col) {
#pragma unroll
          for (int i = 0; i < 8; ++i) lds_val[r * kTileLdsPitch + cpos + i] = v[i];
        }
      } else if (KIND == QK_MX) {
        const uint32_t code = mx_code(group_max4(am));
        const float inv = mx_inv_scale(code);
        const uint32_t w0 = enc_e4m3x4<HW>(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
        const uint32_t w1 = enc_e4m3x4<HW>(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
        if (want_row && grow < rows) {
          *reinterpret_cast<uint2*>(static_cast<uint8_t*>(o.row_q) + grow * o.ld_row + ocol + cpos) =
              make_uint2(w0, w1);
          if ((tid & 3) == 0)
            static_cast<uint8_t*>(o.row_s)[grow * o.rs_row + ((ocol + cpos) >> 5) * o.rs_kb] = uint8_t(code);
        }
        if (want_col) {
#pragma unroll
          for (int i = 0; i < 8; ++i) lds_val[r * kTileLdsPitch + cpos + i] = v[i];
        }
      } else {  // bf16
        if (want_row && grow < rows) {
          const uint4 pk = make_uint4(enc_bf16x2<HW>(v[0], v[1]), enc_bf16x2<HW>(v[2], v[3]),
                                      enc_bf16x2<HW>(v[4], v[5]), enc_bf16x2<HW>(v[6], v[7]));
          *reinterpret_cast<uint4*>(static_cast<uint16_t*>(o.row_q) + grow * o.ld_row + ocol + cpos) = pk;
        }
        if (want_col) {
#pragma unroll
          for (int i = 0; i < 8; ++i) lds_val[r * kTileLdsPitch + cpos + i] = v[i];
        }
      }
    }
    if (!want_col) continue;
    __syncthreads();

    // ---- phase 2: thread -> column c = tid % 128, rows [64*h, 64*h + 64)
    const int c = tid & 127, h = tid >> 7;
    const int64_t gcol = ocol + c;
    uint8_t* qt8 = static_cast<uint8_t*>(o.col_q);
    if (KIND == QK_BLOCK) {
      float am = 0.f;
      for (int r = 0; r < 64; ++r) am = fmaxf(am, fabsf(lds_val[(64 * h + r) * kTileLdsPitch + c]));
      red[h * 128 + c] = am;
      __syncthreads();
      const float s = block_scale(fmaxf(red[c], red[128 + c]), false);
      const float y = 1.0f / s;
      for (int r16 = 0; r16 < 64; r16 += 16) {
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float* p = &lds_val[(64 * h + r16 + 4 * k) * kTileLdsPitch + c];
          w[k] = enc_e4m3x4<HW>(div_rn(p[0], s, y), div_rn(p[kTileLdsPitch], s, y),
                                div_rn(p[2 * kTileLdsPitch], s, y), div_rn(p[3 * kTileLdsPitch], s, y));
        }
        *reinterpret_cast<uint4*>(qt8 + gcol * o.ld_col + row0 + 64 * h + r16) = make_uint4(w[0], w[1], w[2], w[3]);
      }
      if (h == 0) static_cast<float*>(o.col_s)[(row0 >> 7) * o.ld_col_s + gcol] = s;
    } else if (KIND == QK_MX) {
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
            const float* p = &lds_val[(rb + r16 + 4 * k) * kTileLdsPitch + c];
            w[k] = enc_e4m3x4<HW>(p[0] * inv, p[kTileLdsPitch] * inv, p[2 * kTileLdsPitch] * inv,
                                  p[3 * kTileLdsPitch] * inv);
          }
          *reinterpret_cast<uint4*>(qt8 + gcol * o.ld_col + row0 + rb + r16) = make_uint4(w[0], w[1], w[2], w[3]);
        }
        static_cast<uint8_t*>(o.col_s)[((row0 + rb) >> 5) * o.ld_col_s + gcol] = uint8_t(code);
      }
    } else {  // bf16 transpose
      uint16_t* qt16 = static_cast<uint16_t*>(o.col_q);
      for (int r8 = 0; r8 < 64; r8 += 8) {
        const float* p = &lds_val[(64 * h + r8) * kTileLdsPitch + c];
        const uint4 pk = make_uint4(enc_bf16x2<HW>(p[0], p[kTileLdsPitch]),
                                    enc_bf16x2<HW>(p[2 * kTileLdsPitch], p[3 * kTileLdsPitch]),
                                    enc_bf16x2<HW>(p[4 * kTileLdsPitch], p[5 * kTileLdsPitch]),
                                    enc_bf16x2<HW>(p[6 * kTileLdsPitch], p[7 * kTileLdsPitch]));
        *reinterpret_cast<uint4*>(qt16 + gcol * o.ld_col + row0 + 64 * h + r8) = pk;
      }
    }
    if (oi + 1 < NOUT) __syncthreads();  // LDS is reused by the next output
  }
}

// Validates a TileOut against the tile geometry; returns nonzero (with the
// error set) on a mismatch.  `cols` is the source's column count per output.
// TileOut from the C-ABI arguments; `kind` may carry FM_SCALES_KMAJOR.
inline TileOut make_tile_out(int kind, void* q, int64_t ld_q, void* s, int64_t ld_s, void* qt,
                             int64_t ld_qt, void* st, int64_t ld_st, int64_t off0, int64_t off1,
                             const int32_t* tile_valid) {
  const bool kmajor = (kind & FM_SCALES_KMAJOR) != 0;
  TileOut o{kind & ~FM_SCALES_KMAJOR, q, ld_q, s, kmajor ? 1 : ld_s, kmajor ? ld_s : 1,
            qt, ld_qt, st, ld_st, {off0, off1}, tile_valid};
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
  dim3 grid(unsigned(cols / 128), unsigned((rows + 127) / 128));
  switch (o.kind) {
    case QK_BF16: hipLaunchKernelGGL((tile_producer_kernel<Src, QK_BF16>), grid, dim3(256), 0, stream, src, o, rows); break;
    case QK_BLOCK: hipLaunchKernelGGL((tile_producer_kernel<Src, QK_BLOCK>), grid, dim3(256), 0, stream, src, o, rows); break;
    case QK_POW2: hipLaunchKernelGGL((tile_producer_kernel<Src, QK_POW2>), grid, dim3(256), 0, stream, src, o, rows); break;
    default: hipLaunchKernelGGL((tile_producer_kernel<Src, QK_MX>), grid, dim3(256), 0, stream, src, o, rows); break;
  }
  return check_launch(what);
}

}  // namespace fm
