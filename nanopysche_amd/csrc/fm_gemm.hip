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
// Tiling: 256 threads = 4 wave64 as 2 (i) x 2 (j); workgroup tile 256 (i) x
// 128 (j), each wave 128 x 64 = 4 x 2 MFMA 32x32 blocks; K step 128 bytes
// (128 e4m3 / 64 bf16).  Operands and scales stream into a 3-stage LDS ring by
// direct global->LDS loads (see grouped_gemm_kernel).
// Workgroup ids are remapped so each XCD walks a contiguous range of tiles,
// grouped 8 m-tiles at a time for L2 reuse of weights and activations.
#include "fm_common.h"
#include "../../include/fm_hip.h"

namespace fm {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
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

// 16-byte chunk `chunk` of 128-byte row `row` of an operand tile in LDS.  The
// chunk index is XOR-swizzled with (row / 2) % 8: a ds_read_b128 serves 16
// lanes per pass from 64 four-byte banks (two 128-byte rows), and the 16 rows
// those lanes touch then fall on 16 distinct 16-byte bank groups.
__device__ __forceinline__ int lds_swz(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * 128 + ((chunk ^ lds_swz(row)) << 4);
}

__device__ __forceinline__ float scale_f32(const Operand& o, int64_t g, int64_t row, int64_t kb) {
  return static_cast<const float*>(o.s)[g * o.s_gs + (row >> o.s_shift) * o.s_row + kb * o.s_kb];
}
__device__ __forceinline__ uint32_t scale_e8m0(const Operand& o, int64_t g, int64_t row, int64_t kb) {
  return static_cast<const uint8_t*>(o.s)[g * o.s_gs + (row >> o.s_shift) * o.s_row + kb * o.s_kb];
}

// LDS-DMA: the 64 lanes' `size`-byte loads land at consecutive LDS addresses
// starting at `lds` (wave-uniform); `g` is each lane's own global source.
// Issued from inline assembly so the compiler's wait insertion does not treat
// them as pending LDS writes (it would wait for every prefetch in flight before
// each LDS read); the kernel orders them with explicit vmcnt waits instead.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return uint32_t(size_t((__attribute__((address_space(3))) const void*)(p)));
}
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is written here and nowhere else
__device__ __forceinline__ void dma16(const void* g, const void* lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* g, const void* lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(m) : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt bits [3:0] and [15:14],
// expcnt [6:4] left at its maximum, lgkmcnt [11:8]).  Draining lgkmcnt too
// means this wave's LDS reads of a stage have returned before the barrier that
// allows the stage to be refilled.
#define FM_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4))

constexpr int kBI = 256;   // workgroup tile along i (weight rows / M)
constexpr int kBJ = 128;   // workgroup tile along j (tokens / N)

template <int KIND>
struct GemmSmem {
  static constexpr bool kScaled = KIND != GK_BF16;
  static constexpr int kQ = kBI * 128;                 // operand bytes per stage
  static constexpr int kP = kBJ * 128;
  static constexpr int kQS = kScaled ? kBI * 4 : 0;   // scale bytes per stage
  static constexpr int kPS = kScaled ? kBI * 4 : 0;  // 256 slots, the upper 128 unused
  static constexpr int kStage = kQ + kP + kQS + kPS;
};

// Per-lane DMA sources of one workgroup tile.
struct TileSrc {
  const uint8_t* q[8];   // 8 x 1 KiB of the 256-row operand per wave
  const uint8_t* p[4];   // 4 x 1 KiB of the 128-row operand per wave
  const uint8_t* qs;     // scale word of this lane (Q side)
  const uint8_t* ps;     // scale word of this lane (P side; rows past 128 re-read row 127)
  int64_t qs_k, ps_k;    // scale byte advance per K step
};

template <int KIND>
__device__ __forceinline__ void gemm_issue(const TileSrc& src, int64_t k, uint8_t* stage, int wave,
                                           int lane) {
  using SM = GemmSmem<KIND>;
  constexpr int ES = KIND == GK_BF16 ? 2 : 1;
  constexpr int KSTEP = 128 / ES;
  const int64_t kb = k * ES;
#pragma unroll
  for (int u = 0; u < 8; ++u) dma16(src.q[u] + kb, stage + (wave * 8 + u) * 1024);
#pragma unroll
  for (int u = 0; u < 4; ++u) dma16(src.p[u] + kb, stage + SM::kQ + (wave * 4 + u) * 1024);
  if (SM::kScaled) {
    const int64_t ks = k / KSTEP;
    dma4(src.qs + ks * src.qs_k, stage + SM::kQ + SM::kP + wave * 256);
    dma4(src.ps + ks * src.ps_k, stage + SM::kQ + SM::kP + SM::kQS + wave * 256);
  }
}

// One 128-byte K step from a stage: 4 x 2 MFMA 32x32 blocks per wave.
template <int KIND, int MODE>
__device__ __forceinline__ void gemm_compute(const uint8_t* st, v16f (&acc)[4][2], int wi, int wj,
                                             int lrow, int lhalf, bool q_mx_k, bool p_mx_k) {
  using SM = GemmSmem<KIND>;
  const uint8_t* lq = st;
  const uint8_t* lp = st + SM::kQ;
  const float* qs = reinterpret_cast<const float*>(st + SM::kQ + SM::kP);
  const float* ps = reinterpret_cast<const float*>(st + SM::kQ + SM::kP + SM::kQS);
  const uint8_t* qs8 = st + SM::kQ + SM::kP;
  const uint8_t* ps8 = st + SM::kQ + SM::kP + SM::kQS;
  if (KIND == GK_BF16) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      v8bf fa[4], fb[2];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        fa[t] = __builtin_bit_cast(
            v8bf, *reinterpret_cast<const uint4*>(lq + lds_off(wi * 128 + t * 32 + lrow, ks * 2 + lhalf)));
#pragma unroll
      for (int t = 0; t < 2; ++t)
        fb[t] = __builtin_bit_cast(
            v8bf, *reinterpret_cast<const uint4*>(lp + lds_off(wj * 64 + t * 32 + lrow, ks * 2 + lhalf)));
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[a], fb[b], acc[a][b], 0, 0, 0);
    }
    return;
  }
  // 32x32x64 e4m3 fragment: lane half h holds K [16h, 16h+16) in bytes 0-15 and
  // K [32+16h, +16) in bytes 16-31, so bytes 0-15 of both halves form the first
  // 32-deep scale block (scale from lane `row`) and bytes 16-31 the second
  // (scale from lane `row + 32`).
  v8i fa[2][4], fb[2][2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int c0 = ks * 4 + lhalf, c1 = c0 + 2;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = wi * 128 + t * 32 + lrow;
      const uint4 x0 = *reinterpret_cast<const uint4*>(lq + lds_off(r, c0));
      const uint4 x1 = *reinterpret_cast<const uint4*>(lq + lds_off(r, c1));
      fa[ks][t] = v8i{int(x0.x), int(x0.y), int(x0.z), int(x0.w), int(x1.x), int(x1.y), int(x1.z), int(x1.w)};
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r = wj * 64 + t * 32 + lrow;
      const uint4 x0 = *reinterpret_cast<const uint4*>(lp + lds_off(r, c0));
      const uint4 x1 = *reinterpret_cast<const uint4*>(lp + lds_off(r, c1));
      fb[ks][t] = v8i{int(x0.x), int(x0.y), int(x0.z), int(x0.w), int(x1.x), int(x1.y), int(x1.z), int(x1.w)};
    }
  }
  if (KIND == GK_FP8_F32) {
    // 128-deep partial sums, promoted with the product of the block scales
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        v16f part;
#pragma unroll
        for (int r = 0; r < 16; ++r) part[r] = 0.f;
        part = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[0][a], fb[0][b], part, 0, 0, 0, 127, 0, 127);
        part = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[1][a], fb[1][b], part, 0, 0, 0, 127, 0, 127);
        const float sp = ps[wj * 64 + b * 32 + lrow];
        if (MODE == GM_RAGGED_M) {
          const float sc = qs[wi * 128] * sp;  // a wave's 128 rows are one 128x128 weight block
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[a][b][r] += part[r] * sc;
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int ii = wi * 128 + a * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
            acc[a][b][r] += part[r] * (qs[ii] * sp);
          }
        }
      }
    return;
  }
  int sa[2][4], sb[2][2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int blk = ks * 2 + lhalf;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = wi * 128 + t * 32 + lrow;
      if (KIND == GK_FP8_POW2) sa[ks][t] = int((f2u(qs[r]) >> 23) & 0xffu);
      else sa[ks][t] = q_mx_k ? qs8[blk * kBI + r] : qs8[r * 4 + blk];
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r = wj * 64 + t * 32 + lrow;
      if (KIND == GK_FP8_POW2) sb[ks][t] = int((f2u(ps[r]) >> 23) & 0xffu);
      else sb[ks][t] = p_mx_k ? ps8[blk * kBJ + r] : ps8[r * 4 + blk];
    }
  }
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[ks][a], fb[ks][b], acc[a][b], 0, 0,
                                                                   0, sa[ks][a], 0, sb[ks][b]);
}

// Register fragments for one half of a 128-byte K step: for e4m3 one 64-deep
// MFMA K slice (4 A + 2 B fragments of 32 bytes per lane, plus their e8m0
// scale operands), for bf16 two 16-deep slices.
template <int KIND>
struct HalfFrag {
  v8i a[4], b[2];
  int sa[4], sb[2];
};
template <>
struct HalfFrag<GK_BF16> {
  v8bf a[2][4], b[2][2];
};

// Loads half `half` (0 or 1) of the K step held in stage `st`.
template <int KIND>
__device__ __forceinline__ void load_half(const uint8_t* st, int half, HalfFrag<KIND>& f, int wi, int wj,
                                          int lrow, int lhalf, bool q_mx_k, bool p_mx_k) {
  using SM = GemmSmem<KIND>;
  const uint8_t* lq = st;
  const uint8_t* lp = st + SM::kQ;
  if constexpr (KIND == GK_BF16) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int ks = half * 2 + s2;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        f.a[s2][t] = __builtin_bit_cast(
            v8bf, *reinterpret_cast<const uint4*>(lq + lds_off(wi * 128 + t * 32 + lrow, ks * 2 + lhalf)));
#pragma unroll
      for (int t = 0; t < 2; ++t)
        f.b[s2][t] = __builtin_bit_cast(
            v8bf, *reinterpret_cast<const uint4*>(lp + lds_off(wj * 64 + t * 32 + lrow, ks * 2 + lhalf)));
    }
  } else {
    // 32x32x64 e4m3 fragment: lane half h holds K [16h, 16h+16) in bytes 0-15
    // and K [32+16h, +16) in bytes 16-31; bytes 0-15 of both halves form the
    // first 32-deep scale block (scale from lane `row`), bytes 16-31 the second
    // (scale from lane `row + 32`).
    const int c0 = half * 4 + lhalf, c1 = c0 + 2;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = wi * 128 + t * 32 + lrow;
      const v4i x0 = *reinterpret_cast<const v4i*>(lq + lds_off(r, c0));
      const v4i x1 = *reinterpret_cast<const v4i*>(lq + lds_off(r, c1));
      f.a[t] = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r = wj * 64 + t * 32 + lrow;
      const v4i x0 = *reinterpret_cast<const v4i*>(lp + lds_off(r, c0));
      const v4i x1 = *reinterpret_cast<const v4i*>(lp + lds_off(r, c1));
      f.b[t] = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
    }
    const float* qs = reinterpret_cast<const float*>(st + SM::kQ + SM::kP);
    const float* ps = reinterpret_cast<const float*>(st + SM::kQ + SM::kP + SM::kQS);
    const uint8_t* qs8 = st + SM::kQ + SM::kP;
    const uint8_t* ps8 = st + SM::kQ + SM::kP + SM::kQS;
    const int blk = half * 2 + lhalf;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = wi * 128 + t * 32 + lrow;
      if (KIND == GK_FP8_POW2) f.sa[t] = int((f2u(qs[r]) >> 23) & 0xffu);
      else f.sa[t] = q_mx_k ? qs8[blk * kBI + r] : qs8[r * 4 + blk];
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r = wj * 64 + t * 32 + lrow;
      if (KIND == GK_FP8_POW2) f.sb[t] = int((f2u(ps[r]) >> 23) & 0xffu);
      else f.sb[t] = p_mx_k ? ps8[blk * kBJ + r] : ps8[r * 4 + blk];
    }
  }
}

template <int KIND>
__device__ __forceinline__ void mma_half(const HalfFrag<KIND>& f, v16f (&acc)[4][2]) {
  if constexpr (KIND == GK_BF16) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[s2][a], f.b[s2][b], acc[a][b], 0, 0, 0);
  } else {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.a[a], f.b[b], acc[a][b], 0, 0, 0,
                                                                   f.sa[a], 0, f.sb[b]);
  }
}

// Phase C/D of the pipelined loop: refills stage `cur` with K step `k` (the 14
// DMA instructions of gemm_issue) and loads half 0 of the next step from
// `nxt`, two DMAs per group of fragment reads.  The DMAs are inline assembly
// with a memory clobber, so they keep this program order relative to the LDS
// reads, and the MFMA interleave pattern of the caller spreads both between
// the MFMAs instead of queueing all DMAs ahead of them.
template <int KIND>
__device__ __forceinline__ void refill_and_load_half0(const TileSrc& src, int64_t k, uint8_t* cur,
                                                      const uint8_t* nxt, HalfFrag<KIND>& f, int wave,
                                                      int lane, int wi, int wj, int lrow, int lhalf,
                                                      bool q_mx_k, bool p_mx_k) {
  using SM = GemmSmem<KIND>;
  constexpr int ES = KIND == GK_BF16 ? 2 : 1;
  constexpr int KSTEP = 128 / ES;
  const int64_t kb = k * ES;
  const uint8_t* lq = nxt;
  const uint8_t* lp = nxt + SM::kQ;
  if constexpr (KIND == GK_BF16) {
    // half 0 = substeps 0 and 1: A fragments t = 0..3, B fragments t = 0..1
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      dma16(src.q[2 * u] + kb, cur + (wave * 8 + 2 * u) * 1024);
      dma16(src.q[2 * u + 1] + kb, cur + (wave * 8 + 2 * u + 1) * 1024);
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
        f.a[s2][u] = __builtin_bit_cast(
            v8bf, *reinterpret_cast<const uint4*>(lq + lds_off(wi * 128 + u * 32 + lrow, s2 * 2 + lhalf)));
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      dma16(src.p[2 * u] + kb, cur + SM::kQ + (wave * 4 + 2 * u) * 1024);
      dma16(src.p[2 * u + 1] + kb, cur + SM::kQ + (wave * 4 + 2 * u + 1) * 1024);
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
        f.b[s2][u] = __builtin_bit_cast(
            v8bf, *reinterpret_cast<const uint4*>(lp + lds_off(wj * 64 + u * 32 + lrow, s2 * 2 + lhalf)));
    }
  } else {
    const int c0 = lhalf, c1 = c0 + 2;  // half 0
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      dma16(src.q[2 * u] + kb, cur + (wave * 8 + 2 * u) * 1024);
      dma16(src.q[2 * u + 1] + kb, cur + (wave * 8 + 2 * u + 1) * 1024);
      const int r = wi * 128 + u * 32 + lrow;
      const v4i x0 = *reinterpret_cast<const v4i*>(lq + lds_off(r, c0));
      const v4i x1 = *reinterpret_cast<const v4i*>(lq + lds_off(r, c1));
      f.a[u] = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      dma16(src.p[2 * u] + kb, cur + SM::kQ + (wave * 4 + 2 * u) * 1024);
      dma16(src.p[2 * u + 1] + kb, cur + SM::kQ + (wave * 4 + 2 * u + 1) * 1024);
      const int r = wj * 64 + u * 32 + lrow;
      const v4i x0 = *reinterpret_cast<const v4i*>(lp + lds_off(r, c0));
      const v4i x1 = *reinterpret_cast<const v4i*>(lp + lds_off(r, c1));
      f.b[u] = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
    }
    const int64_t ks = k / KSTEP;
    dma4(src.qs + ks * src.qs_k, cur + SM::kQ + SM::kP + wave * 256);
    dma4(src.ps + ks * src.ps_k, cur + SM::kQ + SM::kP + SM::kQS + wave * 256);
    const float* qs = reinterpret_cast<const float*>(nxt + SM::kQ + SM::kP);
    const float* ps = reinterpret_cast<const float*>(nxt + SM::kQ + SM::kP + SM::kQS);
    const uint8_t* qs8 = nxt + SM::kQ + SM::kP;
    const uint8_t* ps8 = nxt + SM::kQ + SM::kP + SM::kQS;
    const int blk = lhalf;  // half 0
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = wi * 128 + t * 32 + lrow;
      if (KIND == GK_FP8_POW2) f.sa[t] = int((f2u(qs[r]) >> 23) & 0xffu);
      else f.sa[t] = q_mx_k ? qs8[blk * kBI + r] : qs8[r * 4 + blk];
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r = wj * 64 + t * 32 + lrow;
      if (KIND == GK_FP8_POW2) f.sb[t] = int((f2u(ps[r]) >> 23) & 0xffu);
      else f.sb[t] = p_mx_k ? ps8[blk * kBJ + r] : ps8[r * 4 + blk];
    }
  }
}

// Scheduling pattern for one half step: each MFMA is followed by LDS reads of
// the next fragments, so the MFMA pipe never waits for operands and the reads
// hide behind the MFMAs (8 x 64-cycle e4m3 MFMAs, or 16 x bf16 MFMAs).
template <int KIND>
__device__ __forceinline__ void interleave_mfma_lds() {
  constexpr int kMfma = KIND == GK_BF16 ? 16 : 8;
  constexpr int kReads = KIND == GK_BF16 ? 1 : 2;
#pragma unroll
  for (int i = 0; i < kMfma; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);  // LDS reads
  }
}

__device__ __forceinline__ void block_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

template <int KIND, int MODE>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(GemmParams p) {
  using SM = GemmSmem<KIND>;
  constexpr int ES = KIND == GK_BF16 ? 2 : 1;         // element size
  constexpr int KSTEP = 128 / ES;                     // elements per 128-byte K step
  constexpr bool SCALED = SM::kScaled;
  constexpr int NLOAD = 12 + (SCALED ? 2 : 0);        // DMA instructions per wave per step
  // three pipeline stages of one K step each (operands + scales)
  __shared__ __attribute__((aligned(1024))) uint8_t smem[3 * SM::kStage];
  uint8_t* const smem0 = smem;
  uint8_t* const smem1 = smem + SM::kStage;
  uint8_t* const smem2 = smem + 2 * SM::kStage;

  // ---------------------------------------------------------- tile decode ----
  const int64_t per_xcd = (p.n_tiles + 7) / 8;
  const int64_t L = int64_t(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (L >= p.n_tiles) return;
  int64_t e, i0, j0, k_lo, k_hi;
  const int64_t NI = (p.n_i + kBI - 1) / kBI;
  if (MODE == GM_RAGGED_M) {
    const int64_t MT = p.m_tiles;
    const int64_t group = L / (kGroupM * NI);
    const int64_t first = group * kGroupM;
    const int64_t gsz = MT - first < kGroupM ? MT - first : kGroupM;
    const int64_t mt = first + (L % gsz);
    const int64_t nt = (L % (kGroupM * NI)) / gsz;
    e = p.tile_expert[mt];
    if (e < 0) return;
    j0 = mt * kBJ;
    i0 = nt * kBI;
    k_lo = 0;
    k_hi = p.K;
  } else {
    const int64_t NJ = p.n_j / kBJ;
    const int64_t per_e = NI * NJ;
    e = L / per_e;
    const int64_t Lr = L % per_e;
    const int64_t group = Lr / (kGroupM * NJ);
    const int64_t first = group * kGroupM;
    const int64_t gsz = NI - first < kGroupM ? NI - first : kGroupM;
    i0 = (first + (Lr % gsz)) * kBI;
    j0 = ((Lr % (kGroupM * NJ)) / gsz) * kBJ;
    k_lo = p.offsets[e];
    k_hi = p.offsets[e + 1];
  }
  if (p.mask != nullptr && p.mask[e] != p.mask_want) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wi = wave >> 1, wj = wave & 1;   // wave tile: i [128*wi, +128), j [64*wj, +64)
  const int lrow = lane & 31, lhalf = lane >> 5;
  const int64_t q_group = MODE == GM_RAGGED_M ? e : 0;
  const int64_t i_last = p.n_i - 1;

  // ------------------------------------------------ per-lane DMA sources ----
  // Linear LDS chunk c = 64*instr + lane of a tile of 128-byte rows holds row
  // c/8, swizzled chunk (c%8) ^ lds_swz(row); each lane fetches the global 16
  // bytes that belong there.  Rows past the end of Q (an N tail) re-read the last row.
  TileSrc src;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int c = (wave * 8 + u) * 64 + lane;
    const int row = c >> 3, ch = (c & 7) ^ lds_swz(row);
    int64_t gr = i0 + row;
    gr = gr < i_last ? gr : i_last;
    src.q[u] = p.Q.p + (q_group * p.Q.gs + gr * p.Q.ld) * ES + ch * 16;
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int c = (wave * 4 + u) * 64 + lane;
    const int row = c >> 3, ch = (c & 7) ^ lds_swz(row);
    src.p[u] = p.P.p + ((j0 + row) * p.P.ld) * ES + ch * 16;
  }
  // Scales: one row per lane, Q 256 rows, P 128 rows (lanes for P rows 128-255
  // re-read row 127 into unused slots, so every wave issues the same loads).
  // MX scales in k-major layout pack four consecutive rows of one 32-block per
  // lane instead ([block][row] bytes in LDS).
  const bool q_mx_k = KIND == GK_FP8_MX && p.Q.s_kb != 1;
  const bool p_mx_k = KIND == GK_FP8_MX && p.P.s_kb != 1;
  src.qs = src.ps = nullptr;
  src.qs_k = src.ps_k = 0;
  if (SCALED) {
    const int qi = wave * 64 + lane;           // 0..255
    const int pi = wave * 64 + lane;           // 0..255, rows >= 128 clamped below
    const int sbytes = KIND == GK_FP8_MX ? 1 : 4;
    if (q_mx_k) {
      const int b = (qi * 4) / kBI, row = (qi * 4) % kBI;
      int64_t gr = i0 + row;
      gr = gr + 3 <= i_last ? gr : i_last - 3;  // n_i is a multiple of 128
      src.qs = static_cast<const uint8_t*>(p.Q.s) + (q_group * p.Q.s_gs + gr * p.Q.s_row + b * p.Q.s_kb);
    } else {
      int64_t gr = i0 + qi;
      gr = gr < i_last ? gr : i_last;
      src.qs = static_cast<const uint8_t*>(p.Q.s) + (q_group * p.Q.s_gs + (gr >> p.Q.s_shift) * p.Q.s_row) * sbytes;
    }
    if (p_mx_k) {
      const int pc = pi < 128 ? pi : 127;      // 4 blocks x 128 rows = 128 lanes of 4 bytes
      const int b = (pc * 4) / kBJ, row = (pc * 4) % kBJ;
      src.ps = static_cast<const uint8_t*>(p.P.s) + ((j0 + row) * p.P.s_row + b * p.P.s_kb);
    } else {
      const int pc = pi < kBJ ? pi : kBJ - 1;
      src.ps = static_cast<const uint8_t*>(p.P.s) + ((j0 + pc) >> p.P.s_shift) * p.P.s_row * sbytes;
    }
    // per K step: one 128-block (fp32 / pow2 scales) or four 32-blocks (MX)
    src.qs_k = (KIND == GK_FP8_MX ? 4 : 1) * p.Q.s_kb * sbytes;
    src.ps_k = (KIND == GK_FP8_MX ? 4 : 1) * p.P.s_kb * sbytes;
  }

  v16f acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  // Pipeline: stage t % 3 is filled two steps ahead.  Readiness of a stage is
  // this wave's own vmcnt wait (DMA writes land in LDS before the counter
  // drops) followed by a barrier; a stage is refilled only after every wave has
  // passed the barrier that follows its last read of it.  The barrier carries
  // no memory fence, which would wait for the prefetches still in flight.
  const int64_t nk = (k_hi - k_lo) / KSTEP;
  if constexpr (KIND == GK_FP8_F32) {
    // fp32 block scales: each 128-deep partial sum is promoted as a whole, so
    // this kind keeps the one-barrier-per-step loop over whole K steps.
    if (nk > 0) gemm_issue<KIND>(src, k_lo, smem0, wave, lane);
    if (nk > 1) gemm_issue<KIND>(src, k_lo + KSTEP, smem1, wave, lane);
    // Main loop: steps with a successor, whose loads are always in flight here,
    // so an unconditional vmcnt(NLOAD) retires exactly the current stage's DMA
    // (the compiler's wait tracking follows it and adds no wait of its own as
    // long as every body issues the same loads).
    int64_t t = 0;
    while (t + 1 < nk) {
  #pragma unroll
      for (int u = 0; u < 3; ++u) {
        if (t + 1 >= nk) break;
        FM_WAIT_VMCNT(NLOAD);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        uint8_t* nxt = u == 0 ? smem2 : (u == 1 ? smem0 : smem1);
        const uint8_t* cur = u == 0 ? smem0 : (u == 1 ? smem1 : smem2);
        // unconditional (keeps the compiler's wait tracking exact): at t = nk-2
        // this re-reads step nk-1 into the stage of step nk, which is never read
        const int64_t tn = t + 2 < nk ? t + 2 : nk - 1;
        gemm_issue<KIND>(src, k_lo + tn * KSTEP, nxt, wave, lane);
        gemm_compute<KIND, MODE>(cur, acc, wi, wj, lrow, lhalf, q_mx_k, p_mx_k);
        ++t;
      }
    }
    if (t < nk) {  // last step: nothing else in flight
      FM_WAIT_VMCNT(0);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      const int sidx = int(t % 3);
      const uint8_t* cur = sidx == 0 ? smem0 : (sidx == 1 ? smem1 : smem2);
      gemm_compute<KIND, MODE>(cur, acc, wi, wj, lrow, lhalf, q_mx_k, p_mx_k);
    }


  } else {
    // Register-pipelined loop.  Every K step t is split in two halves; while
    // the MFMAs of one half run, the fragments of the next half are read:
    //   A  read half 1 of step t          (stage t % 3)
    //   B  MFMAs of half 0 of step t      (registers loaded during step t-1)
    //   C  wait for step t+1's DMA, barrier, refill stage t % 3 with step t+3
    //   D  read half 0 of step t+1        (stage (t+1) % 3)
    //   E  MFMAs of half 1 of step t
    // Each step issues exactly one group of DMA loads (clamped to the last step
    // at the end; the re-read lands in a stage nobody reads again), so
    // vmcnt(NLOAD) always retires exactly step t+1's group at C.
    HalfFrag<KIND> f0, f1;
    if (nk > 0) {
      gemm_issue<KIND>(src, k_lo, smem0, wave, lane);
      gemm_issue<KIND>(src, k_lo + (nk > 1 ? 1 : 0) * KSTEP, smem1, wave, lane);
      gemm_issue<KIND>(src, k_lo + (nk > 2 ? 2 : nk - 1) * KSTEP, smem2, wave, lane);
      FM_WAIT_VMCNT(2 * NLOAD);
      block_barrier();
      load_half<KIND>(smem0, 0, f0, wi, wj, lrow, lhalf, q_mx_k, p_mx_k);
    }
    int cur_off = 0;  // byte offset of stage t % 3
#pragma unroll 1
    for (int64_t t = 0; t < nk; ++t) {
      const int nxt_off = cur_off == 2 * SM::kStage ? 0 : cur_off + SM::kStage;
      uint8_t* cur = smem + cur_off;
      load_half<KIND>(cur, 1, f1, wi, wj, lrow, lhalf, q_mx_k, p_mx_k);   // A
      mma_half<KIND>(f0, acc);                                               // B
      interleave_mfma_lds<KIND>();
      FM_WAIT_VMCNT(NLOAD);                                                  // C
      block_barrier();
      // C+D: refill this stage with step t+3 and read half 0 of step t+1
      // (unconditional: after the last step it reads a stage holding valid data
      // that is never used, which keeps the body one basic block)
      const int64_t tn = t + 3 < nk ? t + 3 : nk - 1;
      refill_and_load_half0<KIND>(src, k_lo + tn * KSTEP, cur, smem + nxt_off, f0, wave, lane, wi, wj,
                                  lrow, lhalf, q_mx_k, p_mx_k);
      mma_half<KIND>(f1, acc);                                               // E
      interleave_mfma_lds<KIND>();
      cur_off = nxt_off;
    }
    FM_WAIT_VMCNT(0);  // no LDS-DMA may still be in flight when the workgroup exits
  }

  // -------------------------------------------------------------- epilogue ----
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int64_t j = j0 + wj * 64 + b * 32 + lrow;
      if (MODE == GM_RAGGED_M) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t i = i0 + wi * 128 + a * 32 + 8 * q + 4 * lhalf;
          if (i >= p.n_i) continue;
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
          const int64_t i = i0 + wi * 128 + a * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
          if (i >= p.n_i) continue;
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
  p.n_tiles = m_tiles * ((N + kBI - 1) / kBI);
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
  p.n_tiles = int64_t(E) * ((M + kBI - 1) / kBI) * (N / kBJ);
  return dispatch_gemm<GM_RAGGED_K>(kind, p, static_cast<hipStream_t>(stream));
}

}  // extern "C"
