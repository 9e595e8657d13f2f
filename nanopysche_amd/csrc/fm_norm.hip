// RMSNorm ahead of the MoE (reference RMSNorm.forward, model/norm.py:32-49, as
// MoEHybridTransformerBlock applies it to the residual stream before routing,
// model/transformer.py:261-263), fused with the activation quantisation:
//   fm_rmsnorm_quantize   y = x * rsqrt(mean(x^2) + eps) * w in fp32, written as
//                         bf16 (the module's output: what the router and the
//                         expert permute read), e4m3 row blocks of those bf16
//                         values with their scales, and the per-row rsqrt for
//                         the backward -- all from one read of x
//   fm_rmsnorm_backward   dx = r g - (r^3 / D) (sum_j g_j x_j) x with g = dy w,
//                         and dw = sum_t dy x r (fp32, per-slice partials in a
//                         caller workspace summed in a fixed order)
// One wave64 owns a row: the row (D = 512 n <= 8192) sits in registers, lane l
// holding columns 512 c + 8 l .. +8, so the sum of squares is one wave
// reduction and each 128-column block (32-column MX block) is the 16 (4)
// consecutive lanes sharing it.  Everything the kernel writes is row-local;
// the 128-token column blocks of the transpose need every row's rsqrt first,
// so they are formed from these outputs (scaling-aware transpose of the row
// blocks, or the column quantiser over y).
#include "fm_tile.h"

namespace fm {
namespace {

__device__ __forceinline__ void ld8(const uint16_t* p, float (&v)[8]) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = u2f(w[j] << 16);
    v[2 * j + 1] = u2f(w[j] & 0xffff0000u);
  }
}
__device__ __forceinline__ void ld8(const float* p, float (&v)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
__device__ __forceinline__ void st8(uint16_t* p, const float (&v)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    w[j] = uint32_t(f32_to_bf16(v[2 * j])) | (uint32_t(f32_to_bf16(v[2 * j + 1])) << 16);
  *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
}
__device__ __forceinline__ void st8(float* p, const float (&v)[8]) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}
__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

struct NormArgs {
  const void* x;
  int64_t ld_x, T, D;
  const void* w;      // [D], bf16 or fp32
  float eps;
  uint16_t* y;        // bf16 [T, ld_y] or null
  int64_t ld_y;
  int kind;           // FM_QUANT_BLOCK / _POW2 / _MX, or -1: no e4m3 output
  uint8_t* q;         // [T, ld_q]
  int64_t ld_q;
  void* s;            // fp32 [T, ld_s >= D/128] or e8m0 [T, ld_s >= D/32]
  int64_t ld_s;
  float* rstd;        // [T] or null
};

template <typename XT, typename WT, int NC>
__global__ __launch_bounds__(256) void rmsnorm_quant_kernel(NormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.T) return;
  const XT* x = static_cast<const XT*>(a.x) + row * a.ld_x + lane * 8;
  float v[NC][8];
#pragma unroll
  for (int c = 0; c < NC; ++c) ld8(x + c * 512, v[c]);
  // variance = mean(x^2) in fp32 (x.float().pow(2).mean(-1))
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = fmaf(v[c][j], v[c][j], ss);
  ss = wave_sum64(ss);
  const float r = 1.0f / sqrtf(ss / float(a.D) + a.eps);
  if (a.rstd && lane == 0) a.rstd[row] = r;
  const WT* w = static_cast<const WT*>(a.w) + lane * 8;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float wv[8];
    ld8(w + c * 512, wv);
    // (x * r) * w, each product rounded to fp32, then to bf16
#pragma unroll
    for (int j = 0; j < 8; ++j) v[c][j] = bf16_to_f32(f32_to_bf16((v[c][j] * r) * wv[j]));
    if (a.y) st8(a.y + row * a.ld_y + c * 512 + lane * 8, v[c]);
  }
  if (a.kind < 0) return;
  // e4m3 row blocks: the block quantisers' exact quotients (a power-of-two
  // reciprocal, or the correctly rounded x / s), encoded by v_cvt_pk_fp8_f32
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[c][j]));
    const int64_t col = c * 512 + lane * 8;
    uint32_t w0, w1;
    if (a.kind == FM_QUANT_MX) {
      m = fmaxf(m, __shfl_xor(m, 1));
      m = fmaxf(m, __shfl_xor(m, 2));
      const uint32_t e = mx_code(m);
      const float inv = mx_inv_scale(e);
      w0 = enc_e4m3x4<true>(v[c][0] * inv, v[c][1] * inv, v[c][2] * inv, v[c][3] * inv);
      w1 = enc_e4m3x4<true>(v[c][4] * inv, v[c][5] * inv, v[c][6] * inv, v[c][7] * inv);
      if ((lane & 3) == 0) static_cast<uint8_t*>(a.s)[row * a.ld_s + col / 32] = uint8_t(e);
    } else {
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
      const float sc = block_scale_dev(m, a.kind == FM_QUANT_POW2);
      if (a.kind == FM_QUANT_POW2) {
        const float inv = pow2_recip(sc);
        w0 = enc_e4m3x4_inrange<true>(v[c][0] * inv, v[c][1] * inv, v[c][2] * inv, v[c][3] * inv);
        w1 = enc_e4m3x4_inrange<true>(v[c][4] * inv, v[c][5] * inv, v[c][6] * inv, v[c][7] * inv);
      } else {
        const Recip d = recip_of(sc);
        w0 = enc_e4m3x4_inrange<true>(div_rn(v[c][0], d), div_rn(v[c][1], d), div_rn(v[c][2], d),
                                      div_rn(v[c][3], d));
        w1 = enc_e4m3x4_inrange<true>(div_rn(v[c][4], d), div_rn(v[c][5], d), div_rn(v[c][6], d),
                                      div_rn(v[c][7], d));
      }
      if ((lane & 15) == 0) static_cast<float*>(a.s)[row * a.ld_s + col / 128] = sc;
    }
    *reinterpret_cast<uint2*>(a.q + row * a.ld_q + col) = make_uint2(w0, w1);
  }
}

// ------------------------------------------------------------ backward ----
// A workgroup (4 waves) owns the rows [slice * rps, +rps) and writes the
// slice's dw partial row to the workspace.  Two shapes:
//  * D <= 1536 (NC <= 3): wave i takes rows i, i + 4, ... whole; each lane
//    keeps its columns' dw partial in registers and the four wave partials
//    are added in wave order through LDS at the end.
//  * larger D: the four waves share each row, wave i holding chunks
//    i, i + 4, ... (columns 512 c + 8 lane .. +8); the row's dot product is
//    the four wave sums added in wave order through LDS (one barrier per row),
//    and each wave's dw partial covers only its own columns, so it writes them
//    directly.  A lane holds at most four chunks of x, dy, w and dw.
// x and dy stay packed in registers and are widened where used.
struct NormBwdArgs {
  const void* dy;
  int64_t ld_dy;
  const void* x;
  int64_t ld_x, T, D;
  const void* w;
  const float* rstd;
  void* dx;            // x's dtype
  int64_t ld_dx;
  float* part;         // [slices, D] or null
  int64_t rps;         // rows per slice
};

template <typename XT>
struct Raw8 {
  uint4 u[sizeof(XT) / 2];
};
template <typename XT>
__device__ __forceinline__ Raw8<XT> ldraw(const XT* p) {
  Raw8<XT> r;
#pragma unroll
  for (int i = 0; i < int(sizeof(XT) / 2); ++i) r.u[i] = reinterpret_cast<const uint4*>(p)[i];
  return r;
}
__device__ __forceinline__ void widen(const Raw8<uint16_t>& r, float (&v)[8]) {
  const uint32_t w[4] = {r.u[0].x, r.u[0].y, r.u[0].z, r.u[0].w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = u2f(w[j] << 16);
    v[2 * j + 1] = u2f(w[j] & 0xffff0000u);
  }
}
__device__ __forceinline__ void widen(const Raw8<float>& r, float (&v)[8]) {
  const uint32_t w[8] = {r.u[0].x, r.u[0].y, r.u[0].z, r.u[0].w, r.u[1].x, r.u[1].y, r.u[1].z, r.u[1].w};
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = u2f(w[j]);
}

// One chunk of a row: dw partial += dy * (x r) and the chunk's share of
// sum_j g_j x_j, g = dy w.
template <typename XT>
__device__ __forceinline__ float chunk_pass1(const Raw8<XT>& xr, const Raw8<XT>& dr, const float (&wc)[8], float r,
                                             float (&pdw)[8]) {
  float xv[8], dv[8];
  widen(xr, xv);
  widen(dr, dv);
  float dot = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    pdw[j] = fmaf(dv[j], xv[j] * r, pdw[j]);
    dot = fmaf(dv[j] * wc[j], xv[j], dot);
  }
  return dot;
}
// dx = r g - k x for one chunk
template <typename XT>
__device__ __forceinline__ void chunk_pass2(const Raw8<XT>& xr, const Raw8<XT>& dr, const float (&wc)[8], float r,
                                            float k, XT* o) {
  float xv[8], dv[8], ov[8];
  widen(xr, xv);
  widen(dr, dv);
#pragma unroll
  for (int j = 0; j < 8; ++j) ov[j] = r * (dv[j] * wc[j]) - k * xv[j];
  st8(o, ov);
}

template <typename XT, typename WT, int NC>
__global__ __launch_bounds__(256) void rmsnorm_bwd_rows_kernel(NormBwdArgs a) {
  __shared__ float4 acc[4][NC * 128];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = int64_t(blockIdx.x) * a.rps;
  const int64_t r1 = r0 + a.rps < a.T ? r0 + a.rps : a.T;
  const float inv_d = 1.0f / float(a.D);
  float wv[NC][8], pdw[NC][8];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    ld8(static_cast<const WT*>(a.w) + c * 512 + lane * 8, wv[c]);
#pragma unroll
    for (int j = 0; j < 8; ++j) pdw[c][j] = 0.f;
  }
  for (int64_t row = r0 + wave; row < r1; row += 4) {
    const XT* xp = static_cast<const XT*>(a.x) + row * a.ld_x + lane * 8;
    const XT* dp = static_cast<const XT*>(a.dy) + row * a.ld_dy + lane * 8;
    Raw8<XT> xr[NC], dr[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      xr[c] = ldraw(xp + c * 512);
      dr[c] = ldraw(dp + c * 512);
    }
    const float r = a.rstd[row];
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) dot += chunk_pass1(xr[c], dr[c], wv[c], r, pdw[c]);
    dot = wave_sum64(dot);
    const float k = ((r * r) * r) * (dot * inv_d);
    XT* o = static_cast<XT*>(a.dx) + row * a.ld_dx + lane * 8;
#pragma unroll
    for (int c = 0; c < NC; ++c) chunk_pass2(xr[c], dr[c], wv[c], r, k, o + c * 512);
  }
  if (a.part == nullptr) return;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    acc[wave][(2 * c) * 64 + lane] = make_float4(pdw[c][0], pdw[c][1], pdw[c][2], pdw[c][3]);
    acc[wave][(2 * c + 1) * 64 + lane] = make_float4(pdw[c][4], pdw[c][5], pdw[c][6], pdw[c][7]);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < NC * 128; i += 256) {
    const float4 p0 = acc[0][i], p1 = acc[1][i], p2 = acc[2][i], p3 = acc[3][i];
    const float4 t = make_float4(((p0.x + p1.x) + p2.x) + p3.x, ((p0.y + p1.y) + p2.y) + p3.y,
                                 ((p0.z + p1.z) + p2.z) + p3.z, ((p0.w + p1.w) + p2.w) + p3.w);
    const int c = i >> 7, h = (i >> 6) & 1, l = i & 63;
    *reinterpret_cast<float4*>(a.part + int64_t(blockIdx.x) * a.D + c * 512 + l * 8 + h * 4) = t;
  }
}

template <typename XT, typename WT, int NC>
__global__ __launch_bounds__(256) void rmsnorm_bwd_split_kernel(NormBwdArgs a) {
  constexpr int CPW = (NC + 3) / 4;   // chunks per wave
  __shared__ float dots[2][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = int64_t(blockIdx.x) * a.rps;
  const int64_t r1 = r0 + a.rps < a.T ? r0 + a.rps : a.T;
  const float inv_d = 1.0f / float(a.D);
  float wv[CPW][8], pdw[CPW][8];
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    const int c = wave + 4 * i;
#pragma unroll
    for (int j = 0; j < 8; ++j) wv[i][j] = pdw[i][j] = 0.f;
    if (c < NC) ld8(static_cast<const WT*>(a.w) + c * 512 + lane * 8, wv[i]);
  }
  int parity = 0;
  for (int64_t row = r0; row < r1; ++row, parity ^= 1) {
    const XT* xp = static_cast<const XT*>(a.x) + row * a.ld_x + lane * 8;
    const XT* dp = static_cast<const XT*>(a.dy) + row * a.ld_dy + lane * 8;
    Raw8<XT> xr[CPW], dr[CPW];
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const int c = wave + 4 * i;
      if (c < NC) {
        xr[i] = ldraw(xp + c * 512);
        dr[i] = ldraw(dp + c * 512);
      }
    }
    const float r = a.rstd[row];
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < CPW; ++i)
      if (wave + 4 * i < NC) dot += chunk_pass1(xr[i], dr[i], wv[i], r, pdw[i]);
    dot = wave_sum64(dot);
    if (lane == 0) dots[parity][wave] = dot;
    __syncthreads();
    dot = ((dots[parity][0] + dots[parity][1]) + dots[parity][2]) + dots[parity][3];
    const float k = ((r * r) * r) * (dot * inv_d);
    XT* o = static_cast<XT*>(a.dx) + row * a.ld_dx + lane * 8;
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const int c = wave + 4 * i;
      if (c < NC) chunk_pass2(xr[i], dr[i], wv[i], r, k, o + c * 512);
    }
  }
  if (a.part == nullptr) return;
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    const int c = wave + 4 * i;
    if (c < NC) st8(a.part + int64_t(blockIdx.x) * a.D + c * 512 + lane * 8, pdw[i]);
  }
}

// dw from the slices' partial rows [slices, D], summed in a fixed order in two
// levels: group g adds slices 32 g .. 32 g + 31 (one wave per 256 columns and
// group), then the group sums are added in four consecutive runs whose totals
// are added in run order.  With one group the first level writes dw.
constexpr int kDwGroup = 32;

__device__ __forceinline__ void store_dw4(void* dw, int dw_f32, int64_t col, const float4& t) {
  if (dw_f32) {
    *reinterpret_cast<float4*>(static_cast<float*>(dw) + col) = t;
  } else {
    uint16_t* o = static_cast<uint16_t*>(dw) + col;
    *reinterpret_cast<uint2*>(o) =
        make_uint2(uint32_t(f32_to_bf16(t.x)) | (uint32_t(f32_to_bf16(t.y)) << 16),
                   uint32_t(f32_to_bf16(t.z)) | (uint32_t(f32_to_bf16(t.w)) << 16));
  }
}

__global__ __launch_bounds__(64) void rmsnorm_dw_groups_kernel(const float* part, int64_t slices, int64_t D,
                                                               float* groups, void* dw, int dw_f32) {
  const int64_t col = int64_t(blockIdx.x) * 256 + threadIdx.x * 4;
  const int64_t s0 = int64_t(blockIdx.y) * kDwGroup;
  const int n = slices - s0 < kDwGroup ? int(slices - s0) : kDwGroup;
  float4 v[kDwGroup];
#pragma unroll
  for (int i = 0; i < kDwGroup; ++i)
    v[i] = i < n ? *reinterpret_cast<const float4*>(part + (s0 + i) * D + col) : make_float4(0.f, 0.f, 0.f, 0.f);
  float4 t = v[0];
#pragma unroll
  for (int i = 1; i < kDwGroup; ++i) {
    t.x += v[i].x;
    t.y += v[i].y;
    t.z += v[i].z;
    t.w += v[i].w;
  }
  if (gridDim.y == 1) store_dw4(dw, dw_f32, col, t);
  else *reinterpret_cast<float4*>(groups + int64_t(blockIdx.y) * D + col) = t;
}

// Second level: four waves per 256 columns, wave w summing groups
// [w q, (w + 1) q) (q = ceil(groups / 4)) in runs of eight loads, the four
// wave sums then added in wave order.
__global__ __launch_bounds__(256) void rmsnorm_dw_final_kernel(const float* groups, int n_groups, int64_t D, void* dw,
                                                               int dw_f32) {
  __shared__ float4 wsum[4][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t col = int64_t(blockIdx.x) * 256 + lane * 4;
  const int q = (n_groups + 3) / 4;
  const int g_lo = wave * q, g_hi = g_lo + q < n_groups ? g_lo + q : n_groups;
  float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int g0 = g_lo; g0 < g_hi; g0 += 8) {
    float4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      v[i] = g0 + i < g_hi ? *reinterpret_cast<const float4*>(groups + int64_t(g0 + i) * D + col)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      t.x += v[i].x;
      t.y += v[i].y;
      t.z += v[i].z;
      t.w += v[i].w;
    }
  }
  wsum[wave][lane] = t;
  __syncthreads();
  if (wave == 0) {
    const float4 a = wsum[0][lane], b = wsum[1][lane], c = wsum[2][lane], d = wsum[3][lane];
    store_dw4(dw, dw_f32, col,
              make_float4(((a.x + b.x) + c.x) + d.x, ((a.y + b.y) + c.y) + d.y, ((a.z + b.z) + c.z) + d.z,
                          ((a.w + b.w) + c.w) + d.w));
  }
}

// D / 512 chunks per lane (D <= 8192)
#define FM_NORM_CHUNKS(X) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(10) X(12) X(14) X(16)

bool norm_d_ok(int64_t D) {
  if (D <= 0 || D % 512) return false;
  switch (D / 512) {
#define FM_NORM_OK(n) case n:
    FM_NORM_CHUNKS(FM_NORM_OK) return true;
#undef FM_NORM_OK
    default: return false;
  }
}

template <typename XT, typename WT>
void launch_fwd(const NormArgs& a, hipStream_t s) {
  const dim3 grid{unsigned((a.T + 3) / 4)}, block{256};
  switch (a.D / 512) {
#define FM_NORM_CASE(n) \
  case n: hipLaunchKernelGGL((rmsnorm_quant_kernel<XT, WT, n>), grid, block, 0, s, a); break;
    FM_NORM_CHUNKS(FM_NORM_CASE)
#undef FM_NORM_CASE
    default: break;
  }
}

template <typename XT, typename WT>
void launch_bwd(const NormBwdArgs& a, int64_t slices, hipStream_t s) {
  const dim3 grid{unsigned(slices)}, block{256};
  switch (a.D / 512) {
#define FM_NORM_CASE(n) \
  case n:                                                                                   \
    if constexpr (n <= 3) hipLaunchKernelGGL((rmsnorm_bwd_rows_kernel<XT, WT, n>), grid, block, 0, s, a); \
    else hipLaunchKernelGGL((rmsnorm_bwd_split_kernel<XT, WT, n>), grid, block, 0, s, a);               \
    break;
    FM_NORM_CHUNKS(FM_NORM_CASE)
#undef FM_NORM_CASE
    default: break;
  }
}

// rows per slice of the backward: at most 1024 slices, at least 8 rows each
int64_t bwd_rows_per_slice(int64_t T) {
  const int64_t rps = (T + 1023) / 1024;
  return rps < 8 ? 8 : rps;
}

}  // namespace
}  // namespace fm

using namespace fm;

extern "C" {

int fm_rmsnorm_quantize(const void* x, int x_dtype, int64_t ld_x, int64_t T, int64_t D, const void* w, int w_dtype,
                        float eps, void* y, int64_t ld_y, int kind, void* q, int64_t ld_q, void* s, int64_t ld_s,
                        float* rstd, void* stream) {
  FM_REQUIRE(T >= 0, "fm_rmsnorm_quantize: negative T");
  FM_REQUIRE(x_dtype == FM_DTYPE_BF16 || x_dtype == FM_DTYPE_F32, "fm_rmsnorm_quantize: x must be bf16 or fp32");
  FM_REQUIRE(w_dtype == FM_DTYPE_BF16 || w_dtype == FM_DTYPE_F32,
             "fm_rmsnorm_quantize: the weight must be bf16 or fp32");
  FM_REQUIRE(norm_d_ok(D), "fm_rmsnorm_quantize: D must be 512 n with n in 1..8, 10, 12, 14 or 16 (got %lld)",
             (long long)D);
  FM_REQUIRE(kind == -1 || kind == FM_QUANT_BLOCK || kind == FM_QUANT_POW2 || kind == FM_QUANT_MX,
             "fm_rmsnorm_quantize: kind must be -1 (no e4m3 output), FM_QUANT_BLOCK, _POW2 or _MX");
  FM_REQUIRE(ld_x >= D && ld_x % 8 == 0, "fm_rmsnorm_quantize: ld_x must be >= D and a multiple of 8");
  FM_REQUIRE(y == nullptr || (ld_y >= D && ld_y % 8 == 0),
             "fm_rmsnorm_quantize: ld_y must be >= D and a multiple of 8");
  FM_REQUIRE(kind == -1 || (ld_q >= D && ld_q % 8 == 0 && ld_s >= D / (kind == FM_QUANT_MX ? 32 : 128)),
             "fm_rmsnorm_quantize: the e4m3 output needs ld_q >= D (a multiple of 8) and ld_s >= D / block");
  if (T == 0) return 0;
  FM_REQUIRE(x != nullptr && w != nullptr, "fm_rmsnorm_quantize: null x or weight");
  FM_REQUIRE(kind == -1 || (q != nullptr && s != nullptr), "fm_rmsnorm_quantize: null q or s");
  const NormArgs a{x, ld_x, T, D, w, eps, static_cast<uint16_t*>(y), ld_y, kind, static_cast<uint8_t*>(q), ld_q,
                   s, ld_s, rstd};
  hipStream_t sm = static_cast<hipStream_t>(stream);
  const bool xb = x_dtype == FM_DTYPE_BF16, wb = w_dtype == FM_DTYPE_BF16;
  if (xb && wb) launch_fwd<uint16_t, uint16_t>(a, sm);
  else if (xb) launch_fwd<uint16_t, float>(a, sm);
  else if (wb) launch_fwd<float, uint16_t>(a, sm);
  else launch_fwd<float, float>(a, sm);
  return check_launch("fm_rmsnorm_quantize");
}

int64_t fm_rmsnorm_backward_workspace_bytes(int64_t T, int64_t D) {
  if (T <= 0 || D <= 0) return 0;
  const int64_t rps = bwd_rows_per_slice(T);
  const int64_t slices = (T + rps - 1) / rps;
  const int64_t groups = (slices + kDwGroup - 1) / kDwGroup;
  return (slices + (groups > 1 ? groups : 0)) * D * int64_t(sizeof(float));
}

int fm_rmsnorm_backward(const void* dy, int64_t ld_dy, const void* x, int x_dtype, int64_t ld_x, int64_t T, int64_t D,
                        const void* w, int w_dtype, const float* rstd, void* dx, int64_t ld_dx, void* dw,
                        int dw_dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  FM_REQUIRE(T >= 0, "fm_rmsnorm_backward: negative T");
  FM_REQUIRE(x_dtype == FM_DTYPE_BF16 || x_dtype == FM_DTYPE_F32, "fm_rmsnorm_backward: x must be bf16 or fp32");
  FM_REQUIRE(w_dtype == FM_DTYPE_BF16 || w_dtype == FM_DTYPE_F32,
             "fm_rmsnorm_backward: the weight must be bf16 or fp32");
  FM_REQUIRE(dw_dtype == FM_DTYPE_BF16 || dw_dtype == FM_DTYPE_F32, "fm_rmsnorm_backward: dw must be bf16 or fp32");
  FM_REQUIRE(norm_d_ok(D), "fm_rmsnorm_backward: D must be 512 n with n in 1..8, 10, 12, 14 or 16 (got %lld)",
             (long long)D);
  FM_REQUIRE(ld_dy >= D && ld_x >= D && ld_dx >= D && ld_dy % 8 == 0 && ld_x % 8 == 0 && ld_dx % 8 == 0,
             "fm_rmsnorm_backward: ld_dy, ld_x and ld_dx must be >= D and multiples of 8");
  FM_REQUIRE(dw == nullptr || (workspace != nullptr && workspace_bytes >= fm_rmsnorm_backward_workspace_bytes(T, D)),
             "fm_rmsnorm_backward: dw needs a workspace of fm_rmsnorm_backward_workspace_bytes(T, D) bytes");
  FM_REQUIRE(T > 0 || dw == nullptr, "fm_rmsnorm_backward: dw of an empty input is zero; the caller clears it");
  if (T == 0) return 0;
  FM_REQUIRE(dy && x && w && rstd && dx, "fm_rmsnorm_backward: null pointer");
  const int64_t rps = bwd_rows_per_slice(T);
  const int64_t slices = (T + rps - 1) / rps;
  const NormBwdArgs a{dy, ld_dy, x, ld_x, T, D, w, rstd, dx, ld_dx, dw ? static_cast<float*>(workspace) : nullptr,
                      rps};
  hipStream_t sm = static_cast<hipStream_t>(stream);
  const bool xb = x_dtype == FM_DTYPE_BF16, wb = w_dtype == FM_DTYPE_BF16;
  if (xb && wb) launch_bwd<uint16_t, uint16_t>(a, slices, sm);
  else if (xb) launch_bwd<uint16_t, float>(a, slices, sm);
  else if (wb) launch_bwd<float, uint16_t>(a, slices, sm);
  else launch_bwd<float, float>(a, slices, sm);
  if (int rc = check_launch("fm_rmsnorm_backward")) return rc;
  if (dw == nullptr) return 0;
  const int64_t groups = (slices + kDwGroup - 1) / kDwGroup;
  float* part = static_cast<float*>(workspace);
  const int f32 = int(dw_dtype == FM_DTYPE_F32);
  hipLaunchKernelGGL(rmsnorm_dw_groups_kernel, dim3(unsigned(D / 256), unsigned(groups)), dim3(64), 0, sm, part,
                     slices, D, part + slices * D, dw, f32);
  if (groups > 1)
    hipLaunchKernelGGL(rmsnorm_dw_final_kernel, dim3(unsigned(D / 256)), dim3(256), 0, sm, part + slices * D,
                       int(groups), D, dw, f32);
  return check_launch("fm_rmsnorm_backward");
}

}  // extern "C"
