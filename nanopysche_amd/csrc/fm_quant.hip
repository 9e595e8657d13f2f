// Blockwise e4m3 quantisation kernels and their C-ABI entry points:
//   fm_quantize            -- 1x128 / 1x32 row blocks, optional fused 128x1 /
//                             32x1 transposed output (one read of the source)
//   fm_quantize_pair       -- fm_quantize of two interleaved expert weight stacks
//                             (gate|up) read in place
//   fm_quantize_weight     -- 128x128 blocks, batched over expert groups, with
//                             optional transposed payload (same blocks)
//   fm_dequantize          -- any block layout -> bf16 / fp32
//   fm_scaling_aware_transpose -- row-quantised e4m3 -> column-quantised e4m3
//                             of the transpose, without the bf16 source
#include "fm_weight_tile.h"

namespace fm {

// Two expert weight stacks a, b = [groups][rows][cols] read as one
// [groups][2 rows][cols] matrix (group g: rows of a, then rows of b), the
// layout of the fused gate|up weight -- without materialising it.
// ALIGNED (rows % 128 == 0): every 128-row tile lies in one matrix, so
// tile_source resolves the matrix and group once per tile and fetch is a
// dense row access; otherwise each fetch maps its row.
template <typename T, bool ALIGNED>
struct PairSrc {
  static constexpr int kOut = 1;
  using Raw = typename DenseSrc<T>::Raw;
  const T* a;
  const T* b;
  int64_t rows, ld;
  const T* tile_base;  // ALIGNED, set by tile_source: logical row r at tile_base + r * ld
  __device__ __forceinline__ Raw fetch(int64_t row, int64_t col) const {
    if constexpr (ALIGNED) {
      return DenseSrc<T>{tile_base, ld}.fetch(row, col);
    } else {
      const int64_t g = row / (2 * rows), r = row % (2 * rows);
      const T* base = r < rows ? a : b;
      return DenseSrc<T>{base + (g * rows + (r < rows ? r : r - rows)) * ld, 0}.fetch(0, col);
    }
  }
  __device__ __forceinline__ void compute(const Raw& r, float v[][8]) const { DenseSrc<T>{}.compute(r, v); }
};
template <typename T>
__device__ __forceinline__ PairSrc<T, true> tile_source(const PairSrc<T, true>& src, int64_t row0) {
  PairSrc<T, true> t = src;
  const int64_t g = row0 / (2 * src.rows), r = row0 - g * 2 * src.rows;
  const T* m = r < src.rows ? src.a : src.b;
  t.tile_base = m + (g * src.rows + (r < src.rows ? r : r - src.rows) - row0) * src.ld;
  return t;
}

template <typename T>
__global__ __launch_bounds__(256) void weight_quant_kernel(WeightQuantArgs a) {
  __shared__ float red[256];
  __shared__ uint32_t tile[128][65];  // [row][col/2] (bf16 pairs) or [row][col/4] (e4m3 quads)
  weight_quant_tile<T>(a, blockIdx.z, blockIdx.y, blockIdx.x, red, tile);
}


template <typename T>
__global__ __launch_bounds__(256) void weight_quant_batch_kernel(WeightQuantBatch b) {
  __shared__ float red[256];
  __shared__ uint32_t tile[128][65];
  const int64_t z = blockIdx.z;
  const int j = int(z / b.groups);
  weight_quant_tile<T>(b.job[j], z - j * b.groups, blockIdx.y, blockIdx.x, red, tile);
}

// ------------------------------------------------------------- dequantise ----
struct DequantArgs {
  const uint8_t* q;
  int64_t rows, cols, ld_q;
  const void* s;        // fp32 or e8m0
  int s_e8m0;
  int row_shift, col_shift;
  int64_t s_row_stride, s_col_stride;
  void* out;            // bf16 or fp32
  int out_f32;
  int64_t ld_out;
};

// grid (column chunks, row groups): thread -> CW consecutive columns of the
// kDequantRows rows of each row group blockIdx.y, blockIdx.y + gridDim.y, ...;
// the CW columns share one scale (CW <= the block width).  A group's loads
// (payload and scales) are all issued before any row is converted.
constexpr int kDequantRows = 4;
template <int CW>
__global__ __launch_bounds__(256) void dequant_kernel(DequantArgs a) {
  constexpr bool HW = FM_HW_CVT != 0;
  constexpr int RPT = kDequantRows;
  const int64_t c = (int64_t(blockIdx.x) * 256 + threadIdx.x) * CW;
  if (c >= a.cols) return;
  for (int64_t rb = int64_t(blockIdx.y) * RPT; rb < a.rows; rb += int64_t(gridDim.y) * RPT) {
    uint32_t wd[RPT][CW / 4];
    float sc[RPT];
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int64_t r = rb + j < a.rows ? rb + j : a.rows - 1;
      if constexpr (CW == 16) {
        const uint4 pk = *reinterpret_cast<const uint4*>(a.q + r * a.ld_q + c);
        wd[j][0] = pk.x; wd[j][1] = pk.y; wd[j][2] = pk.z; wd[j][3] = pk.w;
      } else {
        const uint2 pk = *reinterpret_cast<const uint2*>(a.q + r * a.ld_q + c);
        wd[j][0] = pk.x; wd[j][1] = pk.y;
      }
      const int64_t si = (r >> a.row_shift) * a.s_row_stride + (c >> a.col_shift) * a.s_col_stride;
      sc[j] = a.s_e8m0 ? e8m0_to_f32(static_cast<const uint8_t*>(a.s)[si]) : static_cast<const float*>(a.s)[si];
    }
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int64_t r = rb + j;
      if (r >= a.rows) break;
      float v[CW];
#pragma unroll
      for (int i = 0; i < CW / 4; ++i) {
        if constexpr (HW) {
          hw_dec_e4m3x4(wd[j][i], &v[4 * i]);
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) v[4 * i + k] = e4m3_to_f32(uint8_t(wd[j][i] >> (8 * k)));
        }
      }
#pragma unroll
      for (int i = 0; i < CW; ++i) v[i] *= sc[j];
      if (a.out_f32) {
        float* o = static_cast<float*>(a.out) + r * a.ld_out + c;
#pragma unroll
        for (int i = 0; i < CW / 4; ++i)
          reinterpret_cast<float4*>(o)[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
      } else {
        uint32_t b[CW / 2];
#pragma unroll
        for (int i = 0; i < CW / 2; ++i)
          b[i] = HW ? hw_bf16x2(v[2 * i], v[2 * i + 1])
                    : uint32_t(f32_to_bf16(v[2 * i])) | (uint32_t(f32_to_bf16(v[2 * i + 1])) << 16);
        uint4* o = reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.out) + r * a.ld_out + c);
#pragma unroll
        for (int i = 0; i < CW / 8; ++i) o[i] = make_uint4(b[4 * i], b[4 * i + 1], b[4 * i + 2], b[4 * i + 3]);
      }
    }
  }
}

// --------------------------------------------------- scaling-aware transpose ----
// grid (C/128, R/128).  Column-block scale = largest row scale of the tile;
// qt[c][r] = e4m3(fp32(decode(q[r][c]) * s[r][c/128]) / st).
__global__ __launch_bounds__(256) void sat_kernel(const uint8_t* q, int64_t ld_q, const float* s,
                                                  int64_t ld_s, uint8_t* qt, int64_t ld_qt,
                                                  float* st, int64_t ld_st) {
  __shared__ __attribute__((aligned(16))) uint32_t tile[128 * 33];
  __shared__ float rs[128];
  __shared__ float smax;
  constexpr bool HW = FM_HW_CVT != 0;
  const int tid = threadIdx.x;
  const int64_t r0 = int64_t(blockIdx.y) * 128, c0 = int64_t(blockIdx.x) * 128;
  // load 128x128 bytes: thread -> 16 bytes of rows rr + 32 i (i < 4)
  const int cc = (tid & 7) * 16;
  const int rr = tid >> 3;
  uint4 pk[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) pk[i] = *reinterpret_cast<const uint4*>(q + (r0 + rr + 32 * i) * ld_q + c0 + cc);
  if (tid < 128) rs[tid] = s[(r0 + tid) * ld_s + (c0 >> 7)];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t* t = &tile[code_idx(rr + 32 * i, cc >> 2)];
    t[0] = pk[i].x;
    t[1] = pk[i].y;
    t[2] = pk[i].z;
    t[3] = pk[i].w;
  }
  __syncthreads();
  if (tid < 64) {
    float m = fmaxf(rs[tid], rs[tid + 64]);
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (tid == 0) smax = m;
  }
  __syncthreads();
  const float sc = smax;
  const Recip d = recip_of(sc);
  // each element is e4m3((decode(q) * s_row) / s_col)
  store_transposed_codes(tile, qt, ld_qt, c0, r0, [&](uint32_t word, int row) {
    const float srow = rs[row];
    float f[4];
    if constexpr (HW) {
      hw_dec_e4m3x4(word, f);
    } else {
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) f[c4] = e4m3_to_f32(uint8_t(word >> (8 * c4)));
    }
    // |decode(q) s_row| <= 448 s_row (1 + 2^-24) and s_col >= s_row: within 464
    return enc_e4m3x4_inrange<HW>(div_rn(f[0] * srow, d), div_rn(f[1] * srow, d), div_rn(f[2] * srow, d),
                                  div_rn(f[3] * srow, d));
  });
  if ((tid & 7) == 0) {
    const int cg = tid >> 3;
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) st[(r0 >> 7) * ld_st + c0 + 4 * cg + c4] = sc;
  }
}

// Runs both e4m3 and both bf16 conversion paths on the same inputs.
__global__ __launch_bounds__(256) void convert_check_kernel(const float* x, int64_t n4, uint32_t* e_hw,
                                                            uint32_t* e_sw, uint32_t* b_hw,
                                                            uint32_t* b_sw) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n4; i += int64_t(gridDim.x) * 256) {
    const float4 v = reinterpret_cast<const float4*>(x)[i];
    e_hw[i] = enc_e4m3x4<true>(v.x, v.y, v.z, v.w);
    e_sw[i] = enc_e4m3x4<false>(v.x, v.y, v.z, v.w);
    b_hw[2 * i] = enc_bf16x2<true>(v.x, v.y);
    b_hw[2 * i + 1] = enc_bf16x2<true>(v.z, v.w);
    b_sw[2 * i] = enc_bf16x2<false>(v.x, v.y);
    b_sw[2 * i + 1] = enc_bf16x2<false>(v.z, v.w);
  }
}

// e4m3 -> f32 by the hardware convert and by the integer routine.
__global__ __launch_bounds__(256) void decode_check_kernel(const uint32_t* codes, int64_t n4, float* hw,
                                                           float* sw) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n4; i += int64_t(gridDim.x) * 256) {
    const uint32_t w = codes[i];
    float d[4];
    hw_dec_e4m3x4(w, d);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      hw[4 * i + b] = d[b];
      sw[4 * i + b] = e4m3_to_f32(uint8_t(w >> (8 * b)));
    }
  }
}

// argument checks of one weight job (defined with the entry points)
int check_weight_job(const FmWeightJob& jb);

}  // namespace fm

using namespace fm;

extern "C" {

int fm_decode_check(const void* codes, int64_t n, float* hw, float* sw, void* stream) {
  FM_REQUIRE(codes && hw && sw, "fm_decode_check: null pointer");
  FM_REQUIRE(n % 4 == 0, "fm_decode_check: n must be a multiple of 4");
  if (n == 0) return 0;
  const int64_t n4 = n / 4;
  const unsigned blocks = unsigned(n4 / 256 + 1 < 4096 ? n4 / 256 + 1 : 4096);
  hipLaunchKernelGGL(decode_check_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint32_t*>(codes), n4, hw, sw);
  return check_launch("fm_decode_check");
}

int fm_convert_check(const float* x, int64_t n, void* e4m3_hw, void* e4m3_sw, void* bf16_hw,
                     void* bf16_sw, void* stream) {
  FM_REQUIRE(x && e4m3_hw && e4m3_sw && bf16_hw && bf16_sw, "fm_convert_check: null pointer");
  FM_REQUIRE(n % 4 == 0, "fm_convert_check: n must be a multiple of 4");
  if (n == 0) return 0;
  const int64_t n4 = n / 4;
  const unsigned blocks = unsigned(n4 / 256 + 1 < 4096 ? n4 / 256 + 1 : 4096);
  hipLaunchKernelGGL(convert_check_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     x, n4, static_cast<uint32_t*>(e4m3_hw), static_cast<uint32_t*>(e4m3_sw),
                     static_cast<uint32_t*>(bf16_hw), static_cast<uint32_t*>(bf16_sw));
  return check_launch("fm_convert_check");
}

int fm_quantize(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ld_x, int kind,
                void* q, int64_t ld_q, void* s, int64_t ld_s, void* qt, int64_t ld_qt, void* st,
                int64_t ld_st, void* stream) {
  FM_REQUIRE(x != nullptr, "fm_quantize: null input");
  FM_REQUIRE(x_dtype == FM_DTYPE_BF16 || x_dtype == FM_DTYPE_F32, "fm_quantize: bad input dtype %d",
             x_dtype);
  FM_REQUIRE(ld_x >= cols && ld_x % 8 == 0, "fm_quantize: input pitch must be >= cols and a multiple of 8");
  const TileOut o = make_tile_out(kind, q, ld_q, s, ld_s, qt, ld_qt, st, ld_st, 0, 0, nullptr);
  hipStream_t sm = static_cast<hipStream_t>(stream);
  if (x_dtype == FM_DTYPE_BF16)
    return launch_tile_producer(DenseSrc<uint16_t>{static_cast<const uint16_t*>(x), ld_x}, o, rows,
                                cols, sm, "fm_quantize");
  return launch_tile_producer(DenseSrc<float>{static_cast<const float*>(x), ld_x}, o, rows, cols,
                              sm, "fm_quantize");
}

int fm_quantize_pair(const void* a, const void* b, int dtype, int64_t groups, int64_t rows,
                     int64_t cols, int64_t ld, int kind, void* q, int64_t ld_q, void* s, int64_t ld_s,
                     void* qt, int64_t ld_qt, void* st, int64_t ld_st, void* stream) {
  FM_REQUIRE(a != nullptr && b != nullptr, "fm_quantize_pair: null input");
  FM_REQUIRE(dtype == FM_DTYPE_BF16 || dtype == FM_DTYPE_F32, "fm_quantize_pair: bad input dtype %d", dtype);
  FM_REQUIRE(groups > 0 && rows > 0, "fm_quantize_pair: groups and rows must be positive");
  FM_REQUIRE(ld >= cols && ld % 8 == 0, "fm_quantize_pair: input pitch must be >= cols and a multiple of 8");
  const TileOut o = make_tile_out(kind, q, ld_q, s, ld_s, qt, ld_qt, st, ld_st, 0, 0, nullptr);
  hipStream_t sm = static_cast<hipStream_t>(stream);
  const int64_t total = groups * 2 * rows;
  auto launch = [&](auto tag) {
    using T = decltype(tag);
    const T* pa = static_cast<const T*>(a);
    const T* pb = static_cast<const T*>(b);
    if (rows % 128 == 0)
      return launch_tile_producer(PairSrc<T, true>{pa, pb, rows, ld, nullptr}, o, total, cols, sm, "fm_quantize_pair");
    return launch_tile_producer(PairSrc<T, false>{pa, pb, rows, ld, nullptr}, o, total, cols, sm, "fm_quantize_pair");
  };
  return dtype == FM_DTYPE_BF16 ? launch(uint16_t{}) : launch(float{});
}

int fm_quantize_weight(const void* w, int w_dtype, int64_t groups, int64_t rows, int64_t cols,
                       int64_t ld_w, int64_t gs_w, int kind, void* q, int64_t ld_q, int64_t gs_q,
                       int64_t q_row_off, float* s, int64_t ld_s, int64_t gs_s, void* qt,
                       int64_t ld_qt, int64_t gs_qt, int64_t qt_col_off, float* st, int64_t ld_st,
                       int64_t gs_st, void* stream) {
  const FmWeightJob job{w, w_dtype, groups, rows, cols, ld_w, gs_w, kind, q, ld_q, gs_q, q_row_off,
                        s, ld_s, gs_s, qt, ld_qt, gs_qt, qt_col_off, st, ld_st, gs_st};
  return fm_quantize_weight_batch(&job, 1, stream);
}

int fm_quantize_weight_batch(const FmWeightJob* jobs, int n_jobs, void* stream) {
  WeightSide ws;
  if (int rc = make_weight_side(jobs, n_jobs, ws, "fm_quantize_weight")) return rc;
  const WeightQuantBatch& batch = ws.b;
  const dim3 grid(unsigned(ws.tiles_x), unsigned(ws.tiles_y), unsigned(batch.groups * n_jobs));
  hipStream_t sm = static_cast<hipStream_t>(stream);
  if (n_jobs == 1) {
    if (ws.src_f32) hipLaunchKernelGGL(weight_quant_kernel<float>, grid, dim3(256), 0, sm, batch.job[0]);
    else hipLaunchKernelGGL(weight_quant_kernel<uint16_t>, grid, dim3(256), 0, sm, batch.job[0]);
  } else if (ws.src_f32) {
    hipLaunchKernelGGL(weight_quant_batch_kernel<float>, grid, dim3(256), 0, sm, batch);
  } else {
    hipLaunchKernelGGL(weight_quant_batch_kernel<uint16_t>, grid, dim3(256), 0, sm, batch);
  }
  return check_launch("fm_quantize_weight");
}

}  // extern "C"

namespace fm {
__global__ __launch_bounds__(256) void weight_side_kernel(WeightSide ws) { weight_side_block(ws, blockIdx.x); }

int make_weight_side(const FmWeightJob* jobs, int n_jobs, WeightSide& ws, const char* what) {
  FM_REQUIRE(jobs != nullptr && n_jobs >= 1 && n_jobs <= 4, "%s: 1 to 4 jobs (got %d)", what, n_jobs);
  ws = WeightSide{};
  for (int i = 0; i < n_jobs; ++i) {
    const FmWeightJob& jb = jobs[i];
    if (int rc = check_weight_job(jb)) return rc;
    FM_REQUIRE(jb.groups == jobs[0].groups && jb.rows == jobs[0].rows && jb.cols == jobs[0].cols &&
                   jb.w_dtype == jobs[0].w_dtype,
               "%s: batched jobs must share groups, rows, cols and dtype", what);
    ws.b.job[i] = WeightQuantArgs{jb.w, jb.w_dtype == FM_DTYPE_F32, jb.ld_w, jb.gs_w, jb.kind & ~FM_ROWS_PAIRED,
                                  static_cast<uint8_t*>(jb.q), jb.ld_q, jb.gs_q, jb.q_row_off, jb.s, jb.ld_s,
                                  jb.gs_s, static_cast<uint8_t*>(jb.qt), jb.ld_qt, jb.gs_qt, jb.qt_col_off,
                                  jb.st, jb.ld_st, jb.gs_st, (jb.kind & FM_ROWS_PAIRED) != 0};
  }
  ws.b.groups = jobs[0].groups;
  ws.tiles_x = jobs[0].cols / 128;
  ws.tiles_y = jobs[0].rows / 128;
  ws.total = ws.tiles_x * ws.tiles_y * ws.b.groups * n_jobs;
  ws.src_f32 = jobs[0].w_dtype == FM_DTYPE_F32;
  FM_REQUIRE(ws.total < (int64_t(1) << 31), "%s: %lld weight blocks (at most 2^31 - 1)", what, (long long)ws.total);
  return 0;
}

int launch_weight_side(const WeightSide& ws, int64_t first, int64_t count, hipStream_t s) {
  FM_REQUIRE(first >= 0 && count >= 0 && first + count <= ws.total, "weight blocks [%lld, +%lld) out of %lld",
             (long long)first, (long long)count, (long long)ws.total);
  if (count == 0) return 0;
  FM_REQUIRE(count < (int64_t(1) << 31), "weight blocks: %lld in one launch", (long long)count);
  WeightSide r = ws;
  r.first = first;
  r.count = count;
  hipLaunchKernelGGL(weight_side_kernel, dim3(unsigned(count)), dim3(256), 0, s, r);
  return check_launch("weight blocks");
}

int check_weight_job(const FmWeightJob& jb) {
  const void* w = jb.w;
  const int w_dtype = jb.w_dtype;
  const int64_t groups = jb.groups, rows = jb.rows, cols = jb.cols, ld_w = jb.ld_w, gs_w = jb.gs_w;
  const int kind = jb.kind & ~FM_ROWS_PAIRED;
  const bool paired = (jb.kind & FM_ROWS_PAIRED) != 0;
  const void *q = jb.q, *qt = jb.qt;
  const float *s = jb.s, *st = jb.st;
  const int64_t ld_q = jb.ld_q, q_row_off = jb.q_row_off, ld_qt = jb.ld_qt, qt_col_off = jb.qt_col_off;
  FM_REQUIRE(w != nullptr, "fm_quantize_weight: null input");
  FM_REQUIRE(w_dtype == FM_DTYPE_BF16 || w_dtype == FM_DTYPE_F32, "fm_quantize_weight: bad dtype");
  FM_REQUIRE(kind == QK_BF16 || kind == QK_BLOCK || kind == QK_POW2,
             "fm_quantize_weight: kind must be bf16, block or pow2 (MX weights use fm_quantize)");
  FM_REQUIRE(rows > 0 && cols > 0 && rows % 128 == 0 && cols % 128 == 0,
             "fm_quantize_weight: rows and cols must be positive multiples of 128 (got %lld x %lld)",
             (long long)rows, (long long)cols);
  FM_REQUIRE(groups > 0, "fm_quantize_weight: groups must be positive");
  FM_REQUIRE(q != nullptr || qt != nullptr, "fm_quantize_weight: no output requested");
  FM_REQUIRE(q_row_off % 128 == 0 && qt_col_off % 128 == 0, "fm_quantize_weight: offsets must be multiples of 128");
  if (kind != QK_BF16) {
    FM_REQUIRE(q == nullptr || s != nullptr, "fm_quantize_weight: scale output missing");
    FM_REQUIRE(qt == nullptr || st != nullptr, "fm_quantize_weight: transposed scale output missing");
    FM_REQUIRE(q == nullptr || ld_q % 8 == 0, "fm_quantize_weight: fp8 pitch must be a multiple of 8");
    FM_REQUIRE(qt == nullptr || ld_qt % 16 == 0, "fm_quantize_weight: transposed pitch must be a multiple of 16");
  }
  FM_REQUIRE(ld_w % 8 == 0 && gs_w % 8 == 0, "fm_quantize_weight: source pitch must be a multiple of 8");
  FM_REQUIRE(!paired || (kind != QK_BF16 && ld_q % 64 == 0 && jb.gs_q % (2 * ld_q) == 0),
             "fm_quantize_weight: paired rows need an e4m3 kind, a pitch that is a multiple of 64 and a group "
             "stride of whole row pairs");
  return 0;
}
}  // namespace fm

extern "C" {

int fm_dequantize(const void* q, int64_t rows, int64_t cols, int64_t ld_q, const void* s,
                  int s_e8m0, int row_shift, int col_shift, int64_t s_row_stride,
                  int64_t s_col_stride, void* out, int out_dtype, int64_t ld_out, void* stream) {
  FM_REQUIRE(q != nullptr && s != nullptr && out != nullptr, "fm_dequantize: null pointer");
  FM_REQUIRE(cols % 8 == 0 && ld_q % 8 == 0 && ld_out % 8 == 0,
             "fm_dequantize: cols and pitches must be multiples of 8");
  FM_REQUIRE(col_shift >= 3 && col_shift <= 16 && row_shift >= 0 && row_shift <= 16,
             "fm_dequantize: block shifts out of range");
  FM_REQUIRE(out_dtype == FM_DTYPE_BF16 || out_dtype == FM_DTYPE_F32, "fm_dequantize: bad out dtype");
  if (rows == 0 || cols == 0) return 0;
  DequantArgs a{static_cast<const uint8_t*>(q), rows, cols, ld_q, s, s_e8m0, row_shift, col_shift,
                s_row_stride, s_col_stride, out, out_dtype == FM_DTYPE_F32, ld_out};
  // 16 columns per thread when every 16 share a scale and the pitches allow
  // 16-byte loads, else 8
  const bool wide = col_shift >= 4 && cols % 16 == 0 && ld_q % 16 == 0 && ld_out % 8 == 0 &&
                    (reinterpret_cast<uintptr_t>(q) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  const int cw = wide ? 16 : 8;
  const int64_t groups = (rows + kDequantRows - 1) / kDequantRows;
  const dim3 grid(unsigned((cols / cw + 255) / 256), unsigned(groups < 65535 ? groups : 65535));
  if (wide)
    hipLaunchKernelGGL(dequant_kernel<16>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL(dequant_kernel<8>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("fm_dequantize");
}

int fm_scaling_aware_transpose(const void* q, int64_t rows, int64_t cols, int64_t ld_q,
                               const float* s, int64_t ld_s, void* qt, int64_t ld_qt, float* st,
                               int64_t ld_st, void* stream) {
  FM_REQUIRE(q && s && qt && st, "fm_scaling_aware_transpose: null pointer");
  FM_REQUIRE(rows % 128 == 0 && cols % 128 == 0,
             "fm_scaling_aware_transpose: rows and cols must be multiples of 128 (got %lld x %lld)",
             (long long)rows, (long long)cols);
  FM_REQUIRE(ld_q % 16 == 0 && ld_qt % 16 == 0 && ld_q >= cols && ld_qt >= rows,
             "fm_scaling_aware_transpose: pitches must be multiples of 16 and cover the matrix");
  FM_REQUIRE(ld_s >= cols / 128 && ld_st >= cols, "fm_scaling_aware_transpose: scale pitch too small");
  if (rows == 0 || cols == 0) return 0;
  dim3 grid(unsigned(cols / 128), unsigned(rows / 128));
  hipLaunchKernelGGL(sat_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint8_t*>(q), ld_q, s, ld_s, static_cast<uint8_t*>(qt), ld_qt,
                     st, ld_st);
  return check_launch("fm_scaling_aware_transpose");
}

}  // extern "C"

// ------------------------------------------------------- bandwidth probe ----
// The HBM rates the producers are measured against: a copy with one 4 KiB
// chunk per workgroup (the tile producers' launch shape), a read-only pass
// and a write-only pass, both four 16-byte accesses per lane in flight over
// a grid-stride loop.
namespace fm {
__global__ __launch_bounds__(256) void probe_copy_kernel(const uint4* __restrict__ a, uint4* __restrict__ b) {
  const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
  st_global(b + i, a[i]);
}
__global__ __launch_bounds__(256) void probe_read_kernel(const uint4* __restrict__ a, size_t n,
                                                         uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  for (size_t i = size_t(blockIdx.x) * 1024 + threadIdx.x; i + 768 < n; i += size_t(gridDim.x) * 1024) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = a[i + 256 * u];
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) st_global(sink + threadIdx.x, acc);   // keeps the loads; almost never taken
}
__global__ __launch_bounds__(256) void probe_write_kernel(uint4* __restrict__ b, size_t n) {
  for (size_t i = size_t(blockIdx.x) * 1024 + threadIdx.x; i + 768 < n; i += size_t(gridDim.x) * 1024) {
#pragma unroll
    for (int u = 0; u < 4; ++u) st_global(b + i + 256 * u, make_uint4(u, 1u, 2u, 3u));
  }
}
}  // namespace fm

extern "C" {

int fm_hbm_probe(int kind, const void* src, void* dst, int64_t bytes, void* stream) {
  FM_REQUIRE(kind >= 0 && kind <= 2, "fm_hbm_probe: kind must be 0 (copy), 1 (read) or 2 (write)");
  FM_REQUIRE(bytes > 0 && bytes % 4096 == 0 && bytes / 4096 <= INT32_MAX,
             "fm_hbm_probe: bytes must be a positive multiple of 4096");
  FM_REQUIRE(dst != nullptr && (kind == 2 || src != nullptr), "fm_hbm_probe: null buffer");
  FM_REQUIRE(aligned16(src) && aligned16(dst), "fm_hbm_probe: buffers must be 16-byte aligned");
  const size_t n = size_t(bytes) / 16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (kind == 0) {
    hipLaunchKernelGGL(probe_copy_kernel, dim3(unsigned(n / 256)), dim3(256), 0, s,
                       static_cast<const uint4*>(src), static_cast<uint4*>(dst));
  } else if (kind == 1) {   // dst: at least 1 KiB, written only in the untaken branch
    hipLaunchKernelGGL(probe_read_kernel, dim3(4096), dim3(256), 0, s, static_cast<const uint4*>(src), n,
                       static_cast<uint32_t*>(dst));
  } else {
    hipLaunchKernelGGL(probe_write_kernel, dim3(4096), dim3(256), 0, s, static_cast<uint4*>(dst), n);
  }
  return check_launch("fm_hbm_probe");
}

}  // extern "C"
