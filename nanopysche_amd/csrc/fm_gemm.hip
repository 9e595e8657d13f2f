// Grouped (per-expert) GEMM for the expert block on gfx950 MFMA.
//
// Every product is "NT": both operands are stored K-contiguous,
//   C_tile[i][j] = sum_k Q[i][k] * P[j][k]
// with Q on the MFMA A side (rows i live in accumulator registers) and P on
// the B side (rows j live in lanes).
//
// Modes
//   ragged-M  (forward gate|up and down, dgrad): P = token rows of the padded
//             expert-contiguous buffer, Q = that expert's weight [N, K];
//             output C[token][n].  Each 128-token m-tile belongs to exactly one
//             expert (groups are padded to 128 rows); tile_expert[] maps it.
//   ragged-K  (weight gradients): contraction over the tokens of expert e,
//             Q = [M, tokens] and P = [N, tokens] (column-quantised activations),
//             output C_e[m][n]; rows m >= split go to a second tensor (dW1|dW3).
//
// Arithmetic kinds
//   BF16       v_mfma_f32_32x32x16_bf16
//   FP8_F32    e4m3 with fp32 block scales (1x128 activations, 128x128
//              weights): per 128-deep K block the MFMA partial sum is promoted
//              into the fp32 accumulator with the product of the two scales.
//   FP8_POW2   e4m3 with power-of-two fp32 block scales: the scale exponents go
//              straight into v_mfma_scale_f32_32x32x64_f8f6f4 as e8m0, no
//              promotion.
//   FP8_MX     e4m3 with e8m0 scales per 32 (OCP MXFP8), same instruction.
//
// Tiling: 256 threads = 4 wave64 as 2 (i) x 2 (j); workgroup tile 128 x 128,
// K step 128 bytes (128 e4m3 / 64 bf16); each wave owns 64 x 64 = 2 x 2 MFMA
// 32x32 blocks.  Operands are double-buffered in LDS (2 x 2 x 16 KiB), rows of
// 128 bytes with the 16-byte chunk index XOR-swizzled by (row % 8) so both the
// 16-byte stores and the MFMA fragment reads are bank-conflict free.
// Workgroup ids are remapped so each XCD walks a contiguous range of tiles,
// grouped 8 m-tiles at a time for L2 reuse of weights and activations.
#include "fm_common.h"
#include "../../include/fm_hip.h"

namespace fm {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

enum GemmKind : int { GK_BF16 = 0, GK_FP8_F32 = 1, GK_FP8_POW2 = 2, GK_FP8_MX = 3 };
enum GemmMode : int { GM_RAGGED_M = 0, GM_RAGGED_K = 1 };

struct Operand {
  const uint8_t* p;   // base pointer
  int64_t ld;         // row pitch (elements)
  int64_t gs;         // group stride (elements), ragged-M weights
  const void* s;      // scales: fp32 or e8m0 bytes
  int64_t s_row;      // scale index = g*s_gs + (row >> s_shift)*s_row + kb*s_kb
  int64_t s_kb;       //   kb counts 128-blocks (fp32 / pow2) or 32-blocks (MX)
  int64_t s_gs;
  int s_shift;
};

struct GemmParams {
  Operand P, Q;
  int64_t n_i;        // extent of i (rows of Q per group)
  int64_t n_j;        // ragged-K: extent of j (rows of P)
  int64_t K;          // ragged-M: contraction length
  const int32_t* tile_expert;  // ragged-M
  int64_t m_tiles;             // ragged-M: 128-row tiles in the padded buffer
  const int32_t* offsets;      // ragged-K: [E+1] padded group starts
  int E;
  const int32_t* mask;         // optional per-expert flag; run expert e iff mask[e] == mask_want
  int mask_want;
  void* C;
  int64_t ldC, c_gs;
  void* C2;
  int64_t c2_gs, split;
  int out_f32;
  int64_t n_tiles;    // logical tiles
};

constexpr int kGroupM = 8;

__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * 128 + ((chunk ^ (row & 7)) << 4);
}

__device__ __forceinline__ float scale_f32(const Operand& o, int64_t g, int64_t row, int64_t kb) {
  return static_cast<const float*>(o.s)[g * o.s_gs + (row >> o.s_shift) * o.s_row + kb * o.s_kb];
}
__device__ __forceinline__ uint32_t scale_e8m0(const Operand& o, int64_t g, int64_t row, int64_t kb) {
  return static_cast<const uint8_t*>(o.s)[g * o.s_gs + (row >> o.s_shift) * o.s_row + kb * o.s_kb];
}

template <int KIND, int MODE>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(GemmParams p) {
  constexpr int ES = KIND == GK_BF16 ? 2 : 1;         // element size
  constexpr int KSTEP = 128 / ES;                     // elements per K step
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][128 * 128];  // [stage][Q,P]
  __shared__ float s_lds[2][2][128];                  // fp32 / pow2 scales per row
  __shared__ uint32_t mx_lds[2][2][128];              // 4 e8m0 codes per row per K step

  // ---------------------------------------------------------- tile decode ----
  const int64_t per_xcd = (p.n_tiles + 7) / 8;
  const int64_t L = int64_t(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (L >= p.n_tiles) return;
  int64_t e, i0, j0, k_lo, k_hi;
  {
    const int64_t NI = p.n_i / 128;
    if (MODE == GM_RAGGED_M) {
      const int64_t MT = p.m_tiles;
      const int64_t group = L / (kGroupM * NI);
      const int64_t first = group * kGroupM;
      const int64_t gsz = MT - first < kGroupM ? MT - first : kGroupM;
      const int64_t mt = first + (L % gsz);
      const int64_t nt = (L % (kGroupM * NI)) / gsz;
      e = p.tile_expert[mt];
      if (e < 0) return;
      j0 = mt * 128;
      i0 = nt * 128;
      k_lo = 0;
      k_hi = p.K;
    } else {
      const int64_t NJ = p.n_j / 128;
      const int64_t per_e = NI * NJ;
      e = L / per_e;
      const int64_t Lr = L % per_e;
      const int64_t group = Lr / (kGroupM * NJ);
      const int64_t first = group * kGroupM;
      const int64_t gsz = NI - first < kGroupM ? NI - first : kGroupM;
      i0 = (first + (Lr % gsz)) * 128;
      j0 = ((Lr % (kGroupM * NJ)) / gsz) * 128;
      k_lo = p.offsets[e];
      k_hi = p.offsets[e + 1];
    }
  }
  if (p.mask != nullptr && p.mask[e] != p.mask_want) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wi = wave >> 1, wj = wave & 1;

  // ---------------------------------------------------- global load setup ----
  const int64_t q_group = MODE == GM_RAGGED_M ? e : 0;
  const uint8_t* qbase = p.Q.p + (q_group * p.Q.gs) * ES;
  const uint8_t* pbase = p.P.p;
  uint4 rq[4], rp[4];
  float sq_reg = 0.f, sp_reg = 0.f;
  uint32_t mq_reg = 0, mp_reg = 0;
  const int srow = tid & 127;
  const bool s_is_q = tid < 128;

  auto gload = [&](int64_t k) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int id = tid + 256 * u;
      const int row = id >> 3, c = id & 7;
      rq[u] = *reinterpret_cast<const uint4*>(qbase + ((i0 + row) * p.Q.ld + k) * ES + c * 16);
      rp[u] = *reinterpret_cast<const uint4*>(pbase + ((j0 + row) * p.P.ld + k) * ES + c * 16);
    }
    if (KIND == GK_FP8_F32 || KIND == GK_FP8_POW2) {
      const int64_t kb = k >> 7;
      if (s_is_q) sq_reg = scale_f32(p.Q, q_group, i0 + srow, kb);
      else sp_reg = scale_f32(p.P, 0, j0 + srow, kb);
    } else if (KIND == GK_FP8_MX) {
      const int64_t kb = k >> 5;
      const Operand& o = s_is_q ? p.Q : p.P;
      const int64_t g = s_is_q ? q_group : 0;
      const int64_t row = (s_is_q ? i0 : j0) + srow;
      uint32_t w = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) w |= scale_e8m0(o, g, row, kb + b) << (8 * b);
      if (s_is_q) mq_reg = w; else mp_reg = w;
    }
  };
  auto lstore = [&](int st) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int id = tid + 256 * u;
      const int row = id >> 3, c = id & 7;
      *reinterpret_cast<uint4*>(&lds[st][0][lds_off(row, c)]) = rq[u];
      *reinterpret_cast<uint4*>(&lds[st][1][lds_off(row, c)]) = rp[u];
    }
    if (KIND == GK_FP8_F32 || KIND == GK_FP8_POW2) {
      if (s_is_q) s_lds[st][0][srow] = sq_reg; else s_lds[st][1][srow] = sp_reg;
    } else if (KIND == GK_FP8_MX) {
      if (s_is_q) mx_lds[st][0][srow] = mq_reg; else mx_lds[st][1][srow] = mp_reg;
    }
  };

  v16f acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  const int lrow = lane & 31, lhalf = lane >> 5;
  if (k_lo < k_hi) {
    gload(k_lo);
    lstore(0);
    __syncthreads();
    int st = 0;
    for (int64_t k = k_lo; k < k_hi; k += KSTEP) {
      const bool more = k + KSTEP < k_hi;
      if (more) gload(k + KSTEP);
      const uint8_t* lq = lds[st][0];
      const uint8_t* lp = lds[st][1];
      if (KIND == GK_BF16) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          v8bf fa[2], fb[2];
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const uint4 xa = *reinterpret_cast<const uint4*>(lq + lds_off(wi * 64 + t * 32 + lrow, ks * 2 + lhalf));
            const uint4 xb = *reinterpret_cast<const uint4*>(lp + lds_off(wj * 64 + t * 32 + lrow, ks * 2 + lhalf));
            fa[t] = __builtin_bit_cast(v8bf, xa);
            fb[t] = __builtin_bit_cast(v8bf, xb);
          }
#pragma unroll
          for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
              acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[a], fb[b], acc[a][b], 0, 0, 0);
        }
      } else {
        v8i fa[2][2], fb[2][2];  // [ks][t]
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            // 32x32x64 e4m3 fragment: lane half h holds K [16h, 16h+16) in
            // bytes 0-15 and K [32+16h, 32+16h+16) in bytes 16-31, so bytes
            // 0-15 of both halves form the first 32-deep scale block (scale
            // from lane `row`) and bytes 16-31 the second (lane `row + 32`).
            const int ra = wi * 64 + t * 32 + lrow, rb = wj * 64 + t * 32 + lrow;
            const int c0 = ks * 4 + lhalf, c1 = c0 + 2;
            const uint4 a0 = *reinterpret_cast<const uint4*>(lq + lds_off(ra, c0));
            const uint4 a1 = *reinterpret_cast<const uint4*>(lq + lds_off(ra, c1));
            const uint4 b0 = *reinterpret_cast<const uint4*>(lp + lds_off(rb, c0));
            const uint4 b1 = *reinterpret_cast<const uint4*>(lp + lds_off(rb, c1));
            fa[ks][t] = v8i{int(a0.x), int(a0.y), int(a0.z), int(a0.w), int(a1.x), int(a1.y), int(a1.z), int(a1.w)};
            fb[ks][t] = v8i{int(b0.x), int(b0.y), int(b0.z), int(b0.w), int(b1.x), int(b1.y), int(b1.z), int(b1.w)};
          }
        if (KIND == GK_FP8_F32) {
          // partial sums over this 128-deep block, then promote with the scales
#pragma unroll
          for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b) {
              v16f part;
#pragma unroll
              for (int r = 0; r < 16; ++r) part[r] = 0.f;
              part = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[0][a], fb[0][b], part, 0, 0, 0, 127, 0, 127);
              part = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[1][a], fb[1][b], part, 0, 0, 0, 127, 0, 127);
              const float sp = s_lds[st][1][wj * 64 + b * 32 + lrow];
              if (MODE == GM_RAGGED_M) {
                const float s = s_lds[st][0][0] * sp;  // weight block scale is uniform
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[a][b][r] += part[r] * s;
              } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                  const int ii = wi * 64 + a * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
                  acc[a][b][r] += part[r] * (s_lds[st][0][ii] * sp);
                }
              }
            }
        } else {
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
              for (int b = 0; b < 2; ++b) {
                int sa, sb;
                if (KIND == GK_FP8_POW2) {
                  sa = int((f2u(s_lds[st][0][wi * 64 + a * 32 + lrow]) >> 23) & 0xffu);
                  sb = int((f2u(s_lds[st][1][wj * 64 + b * 32 + lrow]) >> 23) & 0xffu);
                } else {
                  const int sh = 8 * (ks * 2 + lhalf);
                  sa = int((mx_lds[st][0][wi * 64 + a * 32 + lrow] >> sh) & 0xffu);
                  sb = int((mx_lds[st][1][wj * 64 + b * 32 + lrow] >> sh) & 0xffu);
                }
                acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                    fa[ks][a], fb[ks][b], acc[a][b], 0, 0, 0, sa, 0, sb);
              }
        }
      }
      if (more) lstore(st ^ 1);
      __syncthreads();
      st ^= 1;
    }
  }

  // -------------------------------------------------------------- epilogue ----
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int64_t j = j0 + wj * 64 + b * 32 + lrow;
      if (MODE == GM_RAGGED_M) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t i = i0 + wi * 64 + a * 32 + 8 * q + 4 * lhalf;
          if (p.out_f32) {
            float* dst = static_cast<float*>(p.C) + j * p.ldC + i;
            *reinterpret_cast<float4*>(dst) =
                make_float4(acc[a][b][4 * q], acc[a][b][4 * q + 1], acc[a][b][4 * q + 2], acc[a][b][4 * q + 3]);
          } else {
            uint16_t* dst = static_cast<uint16_t*>(p.C) + j * p.ldC + i;
            uint2 w;
            w.x = uint32_t(f32_to_bf16(acc[a][b][4 * q])) | (uint32_t(f32_to_bf16(acc[a][b][4 * q + 1])) << 16);
            w.y = uint32_t(f32_to_bf16(acc[a][b][4 * q + 2])) | (uint32_t(f32_to_bf16(acc[a][b][4 * q + 3])) << 16);
            *reinterpret_cast<uint2*>(dst) = w;
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t i = i0 + wi * 64 + a * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
          const bool second = i >= p.split;
          const int64_t row = second ? i - p.split : i;
          const int64_t off = e * (second ? p.c2_gs : p.c_gs) + row * p.ldC + j;
          void* base = second ? p.C2 : p.C;
          if (p.out_f32) static_cast<float*>(base)[off] = acc[a][b][r];
          else static_cast<uint16_t*>(base)[off] = f32_to_bf16(acc[a][b][r]);
        }
      }
    }
}

template <int KIND, int MODE>
void launch_gemm(const GemmParams& p, hipStream_t s) {
  const int64_t grid = (p.n_tiles + 7) / 8 * 8;
  hipLaunchKernelGGL((grouped_gemm_kernel<KIND, MODE>), dim3(unsigned(grid)), dim3(256), 0, s, p);
}

template <int MODE>
int dispatch_gemm(int kind, const GemmParams& p, hipStream_t s) {
  switch (kind) {
    case GK_BF16: launch_gemm<GK_BF16, MODE>(p, s); break;
    case GK_FP8_F32: launch_gemm<GK_FP8_F32, MODE>(p, s); break;
    case GK_FP8_POW2: launch_gemm<GK_FP8_POW2, MODE>(p, s); break;
    case GK_FP8_MX: launch_gemm<GK_FP8_MX, MODE>(p, s); break;
    default: set_error("grouped gemm: unknown kind %d", kind); return 1;
  }
  return check_launch("grouped gemm");
}

inline Operand make_operand(const FmGemmOperand& o) {
  return Operand{static_cast<const uint8_t*>(o.data), o.ld, o.group_stride, o.scale,
                 o.scale_row_stride, o.scale_kb_stride, o.scale_group_stride, o.scale_row_shift};
}

inline int check_operand(const FmGemmOperand& o, int kind, const char* name) {
  FM_REQUIRE(o.data != nullptr, "grouped gemm: operand %s is null", name);
  FM_REQUIRE(o.ld % 16 == 0, "grouped gemm: operand %s pitch must be a multiple of 16 elements", name);
  FM_REQUIRE(kind == GK_BF16 || o.scale != nullptr, "grouped gemm: operand %s scales are null", name);
  FM_REQUIRE(o.scale_row_shift >= 0 && o.scale_row_shift <= 7, "grouped gemm: operand %s scale_row_shift out of range", name);
  return 0;
}

}  // namespace fm

using namespace fm;

extern "C" {

int fm_grouped_gemm_ragged_m(int kind, const FmGemmOperand* tokens, const FmGemmOperand* weights,
                             int64_t m_tiles, const int32_t* tile_expert, int E, int64_t N,
                             int64_t K, const int32_t* expert_mask, int mask_want, void* out,
                             int out_dtype, int64_t ld_out, void* stream) {
  FM_REQUIRE(tokens && weights && tile_expert && out, "fm_grouped_gemm_ragged_m: null pointer");
  if (int rc = check_operand(*tokens, kind, "tokens")) return rc;
  if (int rc = check_operand(*weights, kind, "weights")) return rc;
  FM_REQUIRE(N > 0 && N % 128 == 0, "fm_grouped_gemm_ragged_m: N must be a positive multiple of 128 (got %lld)", (long long)N);
  FM_REQUIRE(K > 0 && K % 128 == 0, "fm_grouped_gemm_ragged_m: K must be a positive multiple of 128 (got %lld)", (long long)K);
  FM_REQUIRE(E >= 1, "fm_grouped_gemm_ragged_m: E must be >= 1");
  FM_REQUIRE(tokens->ld >= K && weights->ld >= K, "fm_grouped_gemm_ragged_m: operand pitch < K");
  FM_REQUIRE(weights->group_stride >= K, "fm_grouped_gemm_ragged_m: weight group stride < K");
  FM_REQUIRE(ld_out >= N && ld_out % 4 == 0, "fm_grouped_gemm_ragged_m: output pitch must be >= N and a multiple of 4");
  FM_REQUIRE(out_dtype == FM_DTYPE_BF16 || out_dtype == FM_DTYPE_F32, "fm_grouped_gemm_ragged_m: bad out dtype");
  FM_REQUIRE(kind != GK_FP8_F32 || weights->scale_row_shift == 7,
             "fm_grouped_gemm_ragged_m: fp32-scaled weights must use 128-row scale blocks");
  if (m_tiles == 0) return 0;
  GemmParams p{};
  p.P = make_operand(*tokens);
  p.Q = make_operand(*weights);
  p.n_i = N;
  p.K = K;
  p.tile_expert = tile_expert;
  p.m_tiles = m_tiles;
  p.E = E;
  p.mask = expert_mask;
  p.mask_want = mask_want;
  p.C = out;
  p.ldC = ld_out;
  p.out_f32 = out_dtype == FM_DTYPE_F32;
  p.split = INT64_MAX;
  p.n_tiles = m_tiles * (N / 128);
  return dispatch_gemm<GM_RAGGED_M>(kind, p, static_cast<hipStream_t>(stream));
}

int fm_grouped_gemm_ragged_k(int kind, const FmGemmOperand* a_t, const FmGemmOperand* b_t,
                             const int32_t* offsets, int E, int64_t M, int64_t N,
                             const int32_t* expert_mask, int mask_want, void* out, int64_t out_gs,
                             void* out2, int64_t out2_gs, int64_t split_rows, int out_dtype,
                             int64_t ld_out, void* stream) {
  FM_REQUIRE(a_t && b_t && offsets && out, "fm_grouped_gemm_ragged_k: null pointer");
  if (int rc = check_operand(*a_t, kind, "a_t")) return rc;
  if (int rc = check_operand(*b_t, kind, "b_t")) return rc;
  FM_REQUIRE(M > 0 && M % 128 == 0 && N > 0 && N % 128 == 0,
             "fm_grouped_gemm_ragged_k: M and N must be positive multiples of 128 (got %lld x %lld)",
             (long long)M, (long long)N);
  FM_REQUIRE(E >= 1, "fm_grouped_gemm_ragged_k: E must be >= 1");
  FM_REQUIRE(ld_out >= N, "fm_grouped_gemm_ragged_k: output pitch < N");
  FM_REQUIRE(out_dtype == FM_DTYPE_BF16 || out_dtype == FM_DTYPE_F32, "fm_grouped_gemm_ragged_k: bad out dtype");
  FM_REQUIRE(split_rows >= M || (out2 != nullptr && split_rows % 128 == 0 && split_rows > 0),
             "fm_grouped_gemm_ragged_k: split output needs out2 and a 128-aligned split");
  GemmParams p{};
  p.P = make_operand(*b_t);
  p.Q = make_operand(*a_t);
  p.n_i = M;
  p.n_j = N;
  p.offsets = offsets;
  p.E = E;
  p.mask = expert_mask;
  p.mask_want = mask_want;
  p.C = out;
  p.ldC = ld_out;
  p.c_gs = out_gs;
  p.C2 = out2;
  p.c2_gs = out2_gs;
  p.split = split_rows >= M ? INT64_MAX : split_rows;
  p.out_f32 = out_dtype == FM_DTYPE_F32;
  p.n_tiles = int64_t(E) * (M / 128) * (N / 128);
  return dispatch_gemm<GM_RAGGED_K>(kind, p, static_cast<hipStream_t>(stream));
}

}  // extern "C"
