// 128x128 tile producer: one workgroup (256 threads, 4 wave64) turns a
// 128-row x 128-column tile of fp32 values -- produced on the fly by a source
// functor -- into
//   * a row-major output   (bf16, or e4m3 with 1x128 / 1x32 block scales), and/or
//   * a transposed output  (bf16, or e4m3 with 128x1 / 32x1 block scales),
// reading the source exactly once.  HBM-bound: 16-byte loads, 8-byte row
// stores (16 lanes cover one 128-byte row segment), 64-byte transposed stores.
//
// The transposed values go through LDS as fp32 ([128][129] floats, the odd
// pitch keeps column walks conflict-free).
#pragma once

#include "fm_common.h"

namespace fm {

enum QuantKind : int {
  QK_BF16 = 0,   // no quantisation, bf16 payload
  QK_BLOCK = 1,  // e4m3, fp32 scale = amax/448 per 128 block
  QK_POW2 = 2,   // e4m3, power-of-two fp32 scale per 128 block; transposed
                 // output is the scaling-aware transpose of the row output
  QK_MX = 3,     // e4m3, e8m0 scale per 32 block (OCP MX)
};

struct TileOut {
  int kind;              // QuantKind
  // row-major output (nullptr = not wanted)
  void* row_q;           // bf16 or e4m3 [rows, cols] with pitch ld_row (elements)
  int64_t ld_row;
  void* row_s;           // fp32 [rows, cols/128] or e8m0 [rows, cols/32]; pitch ld_row_s
  int64_t ld_row_s;
  // transposed output (nullptr = not wanted); requires rows % 128 == 0
  void* col_q;           // bf16 or e4m3 [cols, rows] with pitch ld_col (elements)
  int64_t ld_col;
  void* col_s;           // fp32 [rows/128, cols] or e8m0 [rows/32, cols]; pitch ld_col_s
  int64_t ld_col_s;
};

constexpr int kTileLdsPitch = 129;

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

__device__ __forceinline__ uint64_t pack8_e4m3(const uint8_t* b) {
  uint64_t r = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) r |= uint64_t(b[i]) << (8 * i);
  return r;
}

// Source functor contract:
//   __device__ void load8(int64_t row, int64_t col, float v[8]) const;
// loads columns [col, col+8) of logical row `row` as fp32 (zeros for rows the
// source treats as padding).  `rows` is the logical row count.
template <class Src>
__device__ __forceinline__ void produce_tile(const Src& src, const TileOut& o, int64_t rows,
                                             int64_t row0, int64_t col0, float* lds,
                                             float* lds_rowscale) {
  const int tid = threadIdx.x;
  const bool want_col = o.col_q != nullptr;
  const bool rowq = o.kind != QK_BF16;
  // ---- phase 1: rows.  thread -> (row = tid/16 + 16*it, 8 columns at 8*(tid%16))
  const int cpos = (tid & 15) * 8;
  // issue all eight 8-column loads before any store so they overlap in flight
  float vv[8][8];
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int64_t grow = row0 + (tid >> 4) + 16 * it;
    if (grow < rows) {
      src.load8(grow, col0 + cpos, vv[it]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) vv[it][i] = 0.f;
    }
  }
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int r = (tid >> 4) + 16 * it;
    const int64_t grow = row0 + r;
    float* v = vv[it];
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(v[i]));
    float keep[8];  // value stored for the transposed pass
#pragma unroll
    for (int i = 0; i < 8; ++i) keep[i] = v[i];
    if (o.kind == QK_BLOCK || o.kind == QK_POW2) {
      const float bam = group_max16(am);
      const float s = block_scale(bam, o.kind == QK_POW2);
      uint8_t q[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = quant_e4m3(v[i], s);
      if (o.kind == QK_POW2) {
        // the transposed output re-expresses the row-quantised values
#pragma unroll
        for (int i = 0; i < 8; ++i) keep[i] = e4m3_to_f32(q[i]) * s;
        if ((tid & 15) == 0) lds_rowscale[r] = s;
      }
      if (o.row_q != nullptr && grow < rows) {
        *reinterpret_cast<uint64_t*>(static_cast<uint8_t*>(o.row_q) + grow * o.ld_row + col0 +
                                     cpos) = pack8_e4m3(q);
        if ((tid & 15) == 0)
          static_cast<float*>(o.row_s)[grow * o.ld_row_s + (col0 >> 7)] = s;
      }
    } else if (o.kind == QK_MX) {
      const float bam = group_max4(am);
      const uint32_t code = mx_code(bam);
      const float inv = mx_inv_scale(code);
      uint8_t q[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = quant_mx(v[i], inv);
      if (o.row_q != nullptr && grow < rows) {
        *reinterpret_cast<uint64_t*>(static_cast<uint8_t*>(o.row_q) + grow * o.ld_row + col0 +
                                     cpos) = pack8_e4m3(q);
        if ((tid & 3) == 0)
          static_cast<uint8_t*>(o.row_s)[grow * o.ld_row_s + ((col0 + cpos) >> 5)] =
              uint8_t(code);
      }
    } else {  // bf16
      if (o.row_q != nullptr && grow < rows) {
        uint16_t b[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) b[i] = f32_to_bf16(v[i]);
        uint4 pk;
        pk.x = uint32_t(b[0]) | (uint32_t(b[1]) << 16);
        pk.y = uint32_t(b[2]) | (uint32_t(b[3]) << 16);
        pk.z = uint32_t(b[4]) | (uint32_t(b[5]) << 16);
        pk.w = uint32_t(b[6]) | (uint32_t(b[7]) << 16);
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(o.row_q) + grow * o.ld_row + col0 +
                                  cpos) = pk;
      }
    }
    (void)rowq;
    if (want_col) {
#pragma unroll
      for (int i = 0; i < 8; ++i) lds[r * kTileLdsPitch + cpos + i] = keep[i];
    }
  }
  if (!want_col) return;
  __syncthreads();
  // ---- phase 2: columns.  thread -> column c = tid % 128, rows [64*h, 64*h+64)
  const int c = tid & 127;
  const int h = tid >> 7;
  float* colmax = lds_rowscale + 128;  // [2][128]
  float am = 0.f;
  if (o.kind == QK_BLOCK) {
    for (int r = 0; r < 64; ++r) am = fmaxf(am, fabsf(lds[(64 * h + r) * kTileLdsPitch + c]));
    colmax[h * 128 + c] = am;
  }
  __syncthreads();
  const int64_t gcol = col0 + c;
  uint8_t* qt8 = static_cast<uint8_t*>(o.col_q);
  if (o.kind == QK_BLOCK || o.kind == QK_POW2) {
    float s;
    if (o.kind == QK_BLOCK) {
      s = block_scale(fmaxf(colmax[c], colmax[128 + c]), false);
    } else {
      s = 0.f;  // largest row scale of the tile (uniform over its columns)
      for (int r = 0; r < 128; ++r) s = fmaxf(s, lds_rowscale[r]);
    }
    for (int r16 = 0; r16 < 64; r16 += 16) {
      uint8_t q[16];
#pragma unroll
      for (int i = 0; i < 16; ++i)
        q[i] = quant_e4m3(lds[(64 * h + r16 + i) * kTileLdsPitch + c], s);
      uint4 pk;
      pk.x = uint32_t(q[0]) | (uint32_t(q[1]) << 8) | (uint32_t(q[2]) << 16) | (uint32_t(q[3]) << 24);
      pk.y = uint32_t(q[4]) | (uint32_t(q[5]) << 8) | (uint32_t(q[6]) << 16) | (uint32_t(q[7]) << 24);
      pk.z = uint32_t(q[8]) | (uint32_t(q[9]) << 8) | (uint32_t(q[10]) << 16) | (uint32_t(q[11]) << 24);
      pk.w = uint32_t(q[12]) | (uint32_t(q[13]) << 8) | (uint32_t(q[14]) << 16) | (uint32_t(q[15]) << 24);
      *reinterpret_cast<uint4*>(qt8 + gcol * o.ld_col + row0 + 64 * h + r16) = pk;
    }
    if (h == 0) static_cast<float*>(o.col_s)[(row0 >> 7) * o.ld_col_s + gcol] = s;
  } else if (o.kind == QK_MX) {
    for (int b = 0; b < 2; ++b) {  // two 32-row MX blocks per thread
      const int rb = 64 * h + 32 * b;
      float m = 0.f;
      for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(lds[(rb + i) * kTileLdsPitch + c]));
      const uint32_t code = mx_code(m);
      const float inv = mx_inv_scale(code);
      for (int r16 = 0; r16 < 32; r16 += 16) {
        uint8_t q[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) q[i] = quant_mx(lds[(rb + r16 + i) * kTileLdsPitch + c], inv);
        uint4 pk;
        pk.x = uint32_t(q[0]) | (uint32_t(q[1]) << 8) | (uint32_t(q[2]) << 16) | (uint32_t(q[3]) << 24);
        pk.y = uint32_t(q[4]) | (uint32_t(q[5]) << 8) | (uint32_t(q[6]) << 16) | (uint32_t(q[7]) << 24);
        pk.z = uint32_t(q[8]) | (uint32_t(q[9]) << 8) | (uint32_t(q[10]) << 16) | (uint32_t(q[11]) << 24);
        pk.w = uint32_t(q[12]) | (uint32_t(q[13]) << 8) | (uint32_t(q[14]) << 16) | (uint32_t(q[15]) << 24);
        *reinterpret_cast<uint4*>(qt8 + gcol * o.ld_col + row0 + rb + r16) = pk;
      }
      static_cast<uint8_t*>(o.col_s)[((row0 + rb) >> 5) * o.ld_col_s + gcol] = uint8_t(code);
    }
  } else {  // bf16 transpose
    uint16_t* qt16 = static_cast<uint16_t*>(o.col_q);
    for (int r8 = 0; r8 < 64; r8 += 8) {
      uint16_t b[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) b[i] = f32_to_bf16(lds[(64 * h + r8 + i) * kTileLdsPitch + c]);
      uint4 pk;
      pk.x = uint32_t(b[0]) | (uint32_t(b[1]) << 16);
      pk.y = uint32_t(b[2]) | (uint32_t(b[3]) << 16);
      pk.z = uint32_t(b[4]) | (uint32_t(b[5]) << 16);
      pk.w = uint32_t(b[6]) | (uint32_t(b[7]) << 16);
      *reinterpret_cast<uint4*>(qt16 + gcol * o.ld_col + row0 + 64 * h + r8) = pk;
    }
  }
}

// Kernel wrapper: grid (cols/128, ceil(rows/128)).  Dynamic LDS is not used;
// the tile buffer is a static array of 128*129 floats + 384 scale slots.
template <class Src>
__global__ __launch_bounds__(256) void tile_producer_kernel(Src src, TileOut o, int64_t rows) {
  __shared__ float lds[128 * kTileLdsPitch];
  __shared__ float lds_rs[128 + 256];
  const int64_t col0 = int64_t(blockIdx.x) * 128;
  const int64_t row0 = int64_t(blockIdx.y) * 128;
  produce_tile(src, o, rows, row0, col0, lds, lds_rs);
}

// Validates a TileOut against the tile geometry; returns nonzero (with the
// error set) on a mismatch.
inline int check_tile_out(const TileOut& o, int64_t rows, int64_t cols) {
  FM_REQUIRE(cols > 0 && cols % 128 == 0, "cols must be a positive multiple of 128 (got %lld)",
             (long long)cols);
  FM_REQUIRE(rows >= 0, "rows must be >= 0");
  FM_REQUIRE(o.kind >= QK_BF16 && o.kind <= QK_MX, "unknown quant kind %d", o.kind);
  FM_REQUIRE(o.row_q != nullptr || o.col_q != nullptr, "no output requested");
  if (o.row_q != nullptr) {
    FM_REQUIRE(o.ld_row >= cols, "row output pitch %lld < cols %lld", (long long)o.ld_row,
               (long long)cols);
    if (o.kind != QK_BF16) {
      FM_REQUIRE(o.row_s != nullptr, "row scale output missing");
      FM_REQUIRE(o.ld_row_s >= (o.kind == QK_MX ? cols / 32 : cols / 128), "row scale pitch too small");
      FM_REQUIRE(o.ld_row % 8 == 0, "fp8 row pitch must be a multiple of 8");
    } else {
      FM_REQUIRE(o.ld_row % 8 == 0, "bf16 row pitch must be a multiple of 8");
    }
  }
  if (o.col_q != nullptr) {
    FM_REQUIRE(rows % 128 == 0, "transposed output needs rows %% 128 == 0 (got %lld)",
               (long long)rows);
    FM_REQUIRE(o.ld_col >= rows, "transposed output pitch too small");
    FM_REQUIRE(o.ld_col % 16 == 0, "transposed output pitch must be a multiple of 16");
    if (o.kind != QK_BF16) {
      FM_REQUIRE(o.col_s != nullptr, "transposed scale output missing");
      FM_REQUIRE(o.ld_col_s >= cols, "transposed scale pitch too small");
    }
  }
  return 0;
}

template <class Src>
int launch_tile_producer(const Src& src, const TileOut& o, int64_t rows, int64_t cols,
                         hipStream_t stream, const char* what) {
  if (int rc = check_tile_out(o, rows, cols)) return rc;
  if (rows == 0) return 0;
  dim3 grid(unsigned(cols / 128), unsigned((rows + 127) / 128));
  hipLaunchKernelGGL(tile_producer_kernel<Src>, grid, dim3(256), 0, stream, src, o, rows);
  return check_launch(what);
}

}  // namespace fm
