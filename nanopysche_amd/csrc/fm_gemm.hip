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
//             output C[token][n].  Groups are padded to 128 rows.
//   ragged-K  (weight gradients): contraction over the tokens of expert e of
//             a_t [M, tokens] and b_t [N, tokens] (column-quantised
//             activations), output C_e[m][n]; rows m >= split go to a second
//             tensor (dW1|dW3).  The 256 x 256 kernel takes P = a_t, Q = b_t
//             (output rows along j, like ragged-M); the fp32-promotion kernel
//             takes Q = a_t, P = b_t.
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
// Two kernels, K step 128 bytes (128 e4m3 / 64 bf16), operands streamed into
// LDS by direct global->LDS loads, each wave 128 x 64 = 4 x 2 MFMA 32x32 blocks:
//   gemm256_kernel  BF16 / FP8_POW2 / FP8_MX.  Tile 256 x 256, 512 threads =
//                   8 wave64 as 2 (i) x 4 (j), two waves per SIMD, two LDS
//                   stages of 66 KiB.  In ragged-M a 256-token tile covers two
//                   128-row groups of one expert; its second half is idle at
//                   an odd group end.
//   gemm_f32_kernel FP8_F32.  Tile 256 x 128, 256 threads = 4 wave64 as
//                   2 x 2, three LDS stages; each 128-deep partial sum is
//                   promoted through a second set of accumulator registers.
// Ragged-M workgroup ids are remapped so each XCD walks a contiguous range of
// the valid tiles, grouped 8 token tiles at a time for L2 reuse of weights and
// activations; within a group the weight tiles vary fastest when an expert's
// weights are small enough to stay cached, so the workgroups running together
// share a few token tiles and cover all the weight tiles: a weight tile is
// fetched from HBM in the first round only, while the token operand, written
// by the kernel just before, is cached in every round (gemm_weight_fast).
// Ragged-K tiles keep launch order (balances uneven experts) unless the
// experts are balanced (contiguous XCD ranges, see decode_tile256).
#include <atomic>
#include <cstdlib>

#include "fm_common.h"
#include <type_traits>
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
  const uint8_t* p2;  // rows at or past `split` of each group: row - split of p2
  int64_t split;      // INT64_MAX: one tensor
};

struct GemmParams {
  Operand P, Q;
  int64_t n_i;        // extent of i (rows of Q per group)
  int64_t n_j;        // ragged-K: extent of j (rows of P)
  int64_t K;          // ragged-M: contraction length
  const int32_t* tile_expert;  // ragged-M, 256 x 128 kernel: expert of each 128-row tile
  int64_t m_tiles;             // ragged-M: 128-row tiles in the padded buffer
  int64_t j_tiles;             // ragged-M, 256 x 256 kernel: bound on 256-row token tiles
  const int32_t* offsets;      // [E+1] padded group starts (rows)
  int E;
  const int32_t* mask;         // optional per-expert flag; run expert e iff mask[e] == mask_want
  int mask_want;
  void* C;
  int64_t ldC, c_gs;
  void* C2;
  int64_t c2_gs, split;
  int out_f32;
  int64_t n_tiles;    // logical tiles
  int rk_xcd;         // ragged-K, 256 x 256 kernels: bit 0 allows the contiguous XCD split, bit 1 the chunked shares
  int splits;         // ragged-K, 256 x 256 kernel: K slices per tile (>1: fp32 partials, C = workspace)
  int64_t ws_slice;   // ragged-K split: elements between the partials of two slices
  int w_fast;         // ragged-M: weight tiles vary fastest within a group of token tiles
  int rk_jfast;       // ragged-K: j tiles (a_t's) vary fastest within a group of i tiles
  int q_nn;           // ragged-M: the weights stored [K][N] (persistent BF16 / FP8 pow2 kernel only)
  int paired;         // ragged-M FP8 pow2, ring kernel: 1 paired tokens (and [N][K] weights), 2 and paired [K][N] weights
};

constexpr int kGroupM = 8;
constexpr bool kRkChunkedDefault = true;

// 16-byte chunk `chunk` of 128-byte row `row` of an operand tile in LDS.  The
// chunk index is XOR-swizzled with (row / 2) % 8: a ds_read_b128 serves 16
// lanes per pass from 64 four-byte banks (two 128-byte rows), and the 16 rows
// those lanes touch then fall on 16 distinct 16-byte bank groups.
__device__ __forceinline__ int lds_swz(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * 128 + ((chunk ^ lds_swz(row)) << 4);
}

// LDS-DMA: the 64 lanes' `size`-byte loads land at consecutive LDS addresses
// starting at `lds` (wave-uniform); `g` is each lane's own global source.
// Issued from inline assembly so the compiler's wait insertion does not treat
// them as pending LDS writes (it would wait for every prefetch in flight before
// each LDS read); the kernels order them with explicit vmcnt waits instead.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return uint32_t(size_t((__attribute__((address_space(3))) const void*)(p)));
}
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is written here and nowhere else
__device__ __forceinline__ void dma16(const void* g, const void* lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m) : "memory", "m0");
}
__device__ __forceinline__ void dma4a(const void* g, uint32_t lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(m) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* g, const void* lds) { dma4a(g, lds_addr(lds)); }
// Buffer-resource form, the 256 x 256 kernel's path: a raw-buffer descriptor
// of a wave-uniform base (the wave's first row of the tile), a 32-bit
// per-lane offset and a 32-bit uniform offset (group + K position), so no
// 64-bit address arithmetic is spent per load.  Measured on gfx950 it moves
// the tile's 64 KiB per K step at the same rate as the flat form.
// byte address = base + voff + soff.
__device__ __forceinline__ void bdma16(v4i rsrc, uint32_t voff, uint32_t soff, uint32_t lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff),
               "s"(m)
               : "memory", "m0");
}
__device__ __forceinline__ void bdma4(v4i rsrc, uint32_t voff, uint32_t soff, uint32_t lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dword %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff),
               "s"(m)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Raw-buffer descriptor (stride 0, no range clipping) of a wave-uniform base.
__device__ __forceinline__ v4i make_rsrc(const void* base) {
  const uint64_t a = uint64_t(size_t(base));
  v4i r;
  r[0] = __builtin_amdgcn_readfirstlane(int(uint32_t(a)));
  r[1] = __builtin_amdgcn_readfirstlane(int(uint32_t(a >> 32) & 0xffffu));
  r[2] = -1;
  r[3] = 0x00020000;   // gfx9 raw buffer: 32-bit data format, no swizzle
  return r;
}

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt bits [3:0] and [15:14],
// expcnt [6:4] left at its maximum, lgkmcnt [11:8]).  Draining lgkmcnt too
// means this wave's LDS reads of a stage have returned before the barrier that
// allows the stage to be refilled.
#define FM_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4))

// A barrier the compiler moves nothing across.  It carries no memory fence,
// which would wait for the prefetches still in flight.
// a >= b for wave-uniform a and b, as a scalar: a select made from it is an
// s_cmp / s_cselect pair.  64-bit comparisons have no scalar form, and a select
// driven by the vector compare needs a VCC -> SCC copy; an exec-mask peephole
// of the compiler has dropped that copy (the select then read a stale SCC and
// wrote every row of a split output to its second tensor).
__device__ __forceinline__ bool uniform_ge(int64_t a, int64_t b) {
  return __builtin_amdgcn_readfirstlane(int(a >= b)) != 0;
}

__device__ __forceinline__ void block_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// ============================================================================
// 256 x 256 kernel: BF16, FP8_POW2, FP8_MX
// ============================================================================
constexpr int kT = 256;

template <int KIND>
struct Smem256 {
  static constexpr bool kScaled = KIND != GK_BF16;
  static constexpr int kOp = kT * 128;                  // one operand, one K step
  static constexpr int kS = kScaled ? kT * 4 : 0;       // its scales
  static constexpr int kP = kOp, kQS = 2 * kOp, kPS = 2 * kOp + kS;
  static constexpr int kStage = 2 * kOp + 2 * kS;
};

// One 256-row operand tile streams as 32 groups of 8 rows x 128 bytes per K
// step, 4 consecutive groups per wave.  LDS chunk c = 64*group + lane holds row
// c/8 at swizzled position c%8, so a lane's global offset inside a group
// depends only on the group's parity.  The valid rows of a tile are a multiple
// of 128, so a wave's 32 rows are all valid or all past the end; a wave past
// the end re-reads the last valid 32 rows into its own LDS rows, which only
// feed outputs that are never stored.
struct OpStream {
  v4i rsrc;               // descriptor of this wave's first row group at K offset 0
  uint32_t group_bytes;   // 8 rows (NN layout: 4 K rows)
  uint32_t lane_off[2];   // even / odd group
  uint32_t k_row_bytes;   // NN layout: bytes per K row (a K step advances 128 of them)
  v4i rsrc2;              // BF16 NN split along K: descriptor of the second tensor
  uint32_t k_split;       //   and the K row it starts at (UINT32_MAX: no split)
};

__device__ __forceinline__ OpStream make_stream(const uint8_t* base, int64_t row_bytes, int64_t rows, int lane,
                                                int wave) {
  OpStream s;
  s.group_bytes = uint32_t(8 * row_bytes);
  const int last = int(rows / 32) - 1;
  s.rsrc = make_rsrc(base + int64_t(wave < last ? wave : last) * 32 * row_bytes);
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int ch = (lane & 7) ^ ((par * 4 + (lane >> 4)) & 7);  // == chunk ^ lds_swz(row)
    s.lane_off[par] = uint32_t((lane >> 3) * row_bytes + ch * 16);
  }
  return s;
}

// e4m3 fragment rows: lane half h holds K [16h, 16h+16) in bytes 0-15 and
// K [32+16h, +16) in bytes 16-31 of the 64-deep slice, so bytes 0-15 of both
// halves form the first 32-deep scale block (scale from lane `row`) and bytes
// 16-31 the second (scale from lane `row + 32`).
__device__ __forceinline__ v8i read_frag8(const uint8_t* base, int r, int half, int lhalf) {
  const int c0 = half * 4 + lhalf;
  const v4i x0 = *reinterpret_cast<const v4i*>(base + lds_off(r, c0));
  const v4i x1 = *reinterpret_cast<const v4i*>(base + lds_off(r, c0 + 2));
  return __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ v8bf read_frag16(const uint8_t* base, int r, int ks, int lhalf) {
  return __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(base + lds_off(r, ks * 2 + lhalf)));
}

// NN weight operand (FP8, stored [K][N]: element (i, k) at k * ld + i).  A K
// step of a 256-row tile is 128 K rows of 256 bytes in LDS, K row k's 16-byte
// chunk c stored at chunk c ^ 2 (k % 8) (32-byte windows rotated by k % 8, so
// the eight K rows one transposed read touches fall on distinct banks).  The
// DMA moves 32 groups of 4 K rows (1 KiB) per step, 4 consecutive groups per
// wave; lane n of a group loads K row n / 16, global chunk (n % 16) ^ 2 k % 8.
__device__ __forceinline__ OpStream make_stream_nn(const uint8_t* base, int64_t ld, int lane, int wave) {
  OpStream s;
  s.group_bytes = uint32_t(4 * ld);
  s.k_row_bytes = uint32_t(ld);
  s.rsrc = make_rsrc(base + int64_t(wave) * 16 * ld);
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int row = lane >> 4, kk = 4 * par + row;
    s.lane_off[par] = uint32_t(row * ld + 16 * ((lane & 15) ^ (2 * kk)));
  }
  return s;
}

// BF16 NN weight operand (stored [K][N]: element (i, k) at k * ld + i).  A K
// step of a 256-row tile is 64 K rows of 512 bytes in LDS, K row k's 16-byte
// chunk c stored at chunk c ^ 4 (k % 4), so the four K rows one transposed
// read touches fall on distinct bank slots.  The DMA moves 32 groups of 2 K
// rows (1 KiB) per step, 4 consecutive groups per wave; lane n of a group
// loads K row n / 32, global chunk (n % 32) ^ 4 (k % 4).
// With a split, K rows from k_split on come from base2 (row k - k_split).
__device__ __forceinline__ OpStream make_stream_nn16(const uint8_t* base, const uint8_t* base2, int64_t k_split,
                                                     int64_t ld_bytes, int lane, int wave) {
  OpStream s;
  s.group_bytes = uint32_t(2 * ld_bytes);
  s.k_row_bytes = uint32_t(ld_bytes);
  s.rsrc = make_rsrc(base + int64_t(wave) * 8 * ld_bytes);
  s.rsrc2 = make_rsrc(base2 + int64_t(wave) * 8 * ld_bytes);
  s.k_split = uint32_t(__builtin_amdgcn_readfirstlane(int(k_split < 0xffffffffll ? k_split : 0xffffffffll)));
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int row = lane >> 5, kk = 2 * par + row;   // k % 4 of the lane's K row
    s.lane_off[par] = uint32_t(row * ld_bytes + 16 * ((lane & 31) ^ (4 * kk)));
  }
  return s;
}

typedef int v2i __attribute__((ext_vector_type(2)));
// ds_read_b64_tr_b8 (gfx950): in each 16-lane group, lanes 2r and 2r + 1 give
// the addresses of bytes 0-7 and 8-15 of row r (r = 0..7), and lane m of the
// group receives byte m of every row (8 bytes, row order).  Established with
// an in-bounds probe of the instruction on the device.
__device__ __forceinline__ v2i lds_read_tr8(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32(
      reinterpret_cast<__attribute__((address_space(3))) v2i*>(
          reinterpret_cast<__attribute__((address_space(3))) uint8_t*>(lds_addr(p))));
}

// NN A fragment of rows ibase + (lane % 32) (ibase a multiple of 32), K half
// `half` of the step: lane l supplies K row 8-block base + (l % 16) / 2 at
// columns ibase + 16 ((l / 16) % 2) + 8 (l % 2), so it receives its own row's
// K bytes [16 h, 16 h + 16) and [32 + 16 h, +16) (h = l / 32) in four reads --
// the byte order of the NT fragment (read_frag8).
__device__ __forceinline__ v8i read_frag8_nn(const uint8_t* st, int ibase, int half, int lane) {
  const int h = lane >> 5, r = (lane >> 1) & 7;
  const int col = (ibase + ((lane >> 4) & 1) * 16 + (lane & 1) * 8) ^ (32 * r);   // every K row read has k % 8 == r
  const uint8_t* b = st + (half * 64 + 16 * h + r) * 256 + col;
  const v2i p0 = lds_read_tr8(b);
  const v2i p1 = lds_read_tr8(b + 8 * 256);
  const v2i p2 = lds_read_tr8(b + 32 * 256);
  const v2i p3 = lds_read_tr8(b + 40 * 256);
  v8i f;
  f[0] = p0[0]; f[1] = p0[1]; f[2] = p1[0]; f[3] = p1[1];
  f[4] = p2[0]; f[5] = p2[1]; f[6] = p3[0]; f[7] = p3[1];
  return f;
}

typedef short v4s16 __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16 (gfx950): in each 16-lane group, lane 4r + p gives the
// address of elements [4p, 4p + 4) of row r (r = 0..3), and lane m of the
// group receives element m of every row (4 elements, row order).  Established
// with an in-bounds probe of the instruction on the device.
__device__ __forceinline__ v4s16 lds_read_tr16(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      reinterpret_cast<__attribute__((address_space(3))) v4s16*>(
          reinterpret_cast<__attribute__((address_space(3))) uint8_t*>(lds_addr(p))));
}

// BF16 NN A fragment of rows ibase + (lane % 32) (ibase a multiple of 32), K
// slice ks (16 deep) of the step: lane half h = lane / 32 takes K [16 ks + 8 h,
// +8) of its row as two reads of four K rows -- the element order of
// read_frag16.  Every K row a lane addresses has k % 4 == r = (lane % 16) / 4.
__device__ __forceinline__ v8bf read_frag16_nn(const uint8_t* st, int ibase, int ks, int lane) {
  const int m = lane & 15, r = m >> 2;
  const int col = ibase + ((lane >> 4) & 1) * 16 + (m & 3) * 4;
  const int k = 16 * ks + 8 * (lane >> 5) + r;
  const uint8_t* b = st + k * 512 + (((col >> 3) ^ (4 * r)) << 4) + (col & 7) * 2;
  const v4s16 lo = lds_read_tr16(b);
  const v4s16 hi = lds_read_tr16(b + 4 * 512);
  return __builtin_bit_cast(v8bf, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Scales in LDS.  pow2: the DMA places the fp32 scale of tile row
// 128*w + 32*t + l at float index 128*w + 4*l + t, so the four row blocks t of
// a lane's fragment rows come from one 16-byte read per K step (both halves
// use them).  MX: four e8m0 bytes per row and step, [block][row] bytes in the
// k-major layout, [row][block] otherwise; read per half.
__device__ __forceinline__ int scale_row_slot(int li) {   // LDS slot li holds tile row:
  return (li >> 7) * 128 + (li & 3) * 32 + ((li & 127) >> 2);
}
// pow2 scales reach the MFMA packed: the e8m0 exponents of a lane's four row
// blocks are the four bytes of one register (positive power-of-two floats: the
// exponent is bits 23-30), and each MFMA selects its byte with op_sel.
__device__ __forceinline__ int pack_exp4(uint32_t x, uint32_t y, uint32_t z, uint32_t w) {
  return int((x >> 23) | ((y >> 23) << 8) | ((z >> 23) << 16) | ((w >> 23) << 24));
}
__device__ __forceinline__ int read_pow2_scales(const uint8_t* st, int off, int w128, int lrow) {
  const uint4 v = *reinterpret_cast<const uint4*>(st + off + (w128 + lrow * 4) * 4);
  return pack_exp4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ int read_mx_scale(const uint8_t* st, int off, int r, int blk, bool mx_k) {
  return mx_k ? st[off + blk * kT + r] : st[off + r * 4 + blk];
}

// Per-lane scale source of one operand: descriptor of the operand's scales
// (group base, wave-uniform), this lane's byte offset at K offset 0, byte
// advance per K step, LDS byte offset of the slot.  fp32 / pow2 and row-major
// MX: one row per slot (pow2 slots permuted, see scale_row_slot); MX in
// k-major layout: four consecutive rows of one 32-block per slot ([block][row]
// bytes in LDS).  Rows past the valid ones re-read the last one.
struct ScaleSrc {
  v4i rsrc;
  uint32_t voff;
  uint32_t k;
  int dst;
};

template <int KIND>
__device__ __forceinline__ ScaleSrc make_scale_src(const Operand& o, int64_t r0, int64_t rows, int64_t og,
                                                   bool mx_k, int li, int lds_base) {
  ScaleSrc s;
  const int sbytes = KIND == GK_FP8_MX ? 1 : 4;
  s.rsrc = make_rsrc(static_cast<const uint8_t*>(o.s) + og * o.s_gs * sbytes);
  if (mx_k) {
    int64_t gr = r0 + (li * 4) % kT;
    gr = gr + 4 <= r0 + rows ? gr : r0 + rows - 4;
    s.voff = uint32_t(gr * o.s_row + (li / 64) * o.s_kb);
  } else {
    const int lr = KIND == GK_FP8_POW2 ? scale_row_slot(li) : li;
    const int64_t gr = r0 + (lr < rows ? lr : rows - 1);
    s.voff = uint32_t((gr >> o.s_shift) * o.s_row * sbytes);
  }
  s.k = uint32_t((KIND == GK_FP8_MX ? 4 : 1) * o.s_kb * sbytes);
  s.dst = lds_base + li * 4;
  return s;
}

// Waves as 2 (i) x 4 (j), each 128 x 64 = 4 x 2 MFMA blocks (128 accumulator
// registers), so two waves share each SIMD: while one waits on LDS reads or
// the per-step barrier the other keeps the matrix pipe busy.  Each wave
// streams 4 of the 32 row groups of each operand and one dword of scales per
// K step.
template <int KIND>
struct Frag {
  v8i a[4], b[2];
  // e8m0 scales of the 4 (a) and 2 (b) row blocks: one register each for MX,
  // packed one byte each into sa[0] / sb[0] for pow2
  int sa[KIND == GK_FP8_MX ? 4 : 1], sb[KIND == GK_FP8_MX ? 2 : 1];
};
template <>
struct Frag<GK_BF16> {
  v8bf a[2][4], b[2][2];
};

struct WaveCoord {
  int wave, lane, wi, wj, lrow, lhalf;
  bool q_mx_k, p_mx_k;
};

// The weight operand's descriptor and uniform byte offset for K step k (kb:
// its byte offset in the NT layout): BF16 [K][N] weights split along K take
// the rows from k_split on from the second tensor (a step never straddles it).
template <int KIND, bool QNN>
__device__ __forceinline__ void q_source(const OpStream& qst, int64_t k, uint32_t kb, v4i& rs, uint32_t& kq) {
  if constexpr (QNN && KIND == GK_BF16) {
    const bool second = uint32_t(k) >= qst.k_split;
    rs = second ? qst.rsrc2 : qst.rsrc;
    kq = (second ? uint32_t(k) - qst.k_split : uint32_t(k)) * qst.k_row_bytes;
  } else {
    rs = qst.rsrc;
    kq = QNN ? uint32_t(k) * qst.k_row_bytes : kb;
  }
}

// One K step of DMA for this wave: 4 row groups of each operand, then one
// scale dword per lane (waves 0-3: Q scale slots, 4-7: P scale slots).
template <int KIND, bool QNN = false>
__device__ __forceinline__ void issue_step(const OpStream& qst, const OpStream& pst, const ScaleSrc& sc, int64_t k,
                                           uint32_t dst, int wave) {
  using SM = Smem256<KIND>;
  constexpr int ES = KIND == GK_BF16 ? 2 : 1;
  constexpr int KSTEP = 128 / ES;
  const uint32_t kb = uint32_t(k * ES);
  v4i qrs;
  uint32_t kq;
  q_source<KIND, QNN>(qst, k, kb, qrs, kq);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    bdma16(qrs, qst.lane_off[u & 1], u * qst.group_bytes + kq, dst + (wave * 4 + u) * 1024);
    bdma16(pst.rsrc, pst.lane_off[u & 1], u * pst.group_bytes + kb, dst + SM::kP + (wave * 4 + u) * 1024);
  }
  if constexpr (KIND != GK_BF16) bdma4(sc.rsrc, sc.voff, uint32_t((k / KSTEP) * sc.k), dst + sc.dst);
}

// Reads half `half` of the K step in stage `st` (pow2 scales only for half 0:
// one scale per 128-deep step).
template <int KIND, bool QNN = false>
__device__ __forceinline__ void read_half(const uint8_t* st, int half, Frag<KIND>& f, const WaveCoord& w) {
  using SM = Smem256<KIND>;
  if constexpr (KIND == GK_BF16) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        if constexpr (QNN) f.a[s2][t] = read_frag16_nn(st, w.wi * 128 + t * 32, half * 2 + s2, w.lane);
        else f.a[s2][t] = read_frag16(st, w.wi * 128 + t * 32 + w.lrow, half * 2 + s2, w.lhalf);
        if (t < 2) f.b[s2][t] = read_frag16(st + SM::kP, w.wj * 64 + t * 32 + w.lrow, half * 2 + s2, w.lhalf);
      }
  } else {
    if constexpr (KIND == GK_FP8_MX) {   // scales first: the MFMAs wait on them
      const int blk = half * 2 + w.lhalf;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f.sa[t] = read_mx_scale(st, SM::kQS, w.wi * 128 + t * 32 + w.lrow, blk, w.q_mx_k);
        if (t < 2) f.sb[t] = read_mx_scale(st, SM::kPS, w.wj * 64 + t * 32 + w.lrow, blk, w.p_mx_k);
      }
    } else if (half == 0) {
      f.sa[0] = read_pow2_scales(st, SM::kQS, w.wi * 128, w.lrow);
      // P rows 64*wj + 32*t + l sit in 128-row block wj/2 at slot t' = 2*(wj&1) + t
      const uint2 v = *reinterpret_cast<const uint2*>(
          st + SM::kPS + ((w.wj >> 1) * 128 + w.lrow * 4 + 2 * (w.wj & 1)) * 4);
      f.sb[0] = pack_exp4(v.x, v.y, 0u, 0u);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if constexpr (QNN) f.a[t] = read_frag8_nn(st, w.wi * 128 + t * 32, half, w.lane);
      else f.a[t] = read_frag8(st, w.wi * 128 + t * 32 + w.lrow, half, w.lhalf);
      if (t < 2) f.b[t] = read_frag8(st + SM::kP, w.wj * 64 + t * 32 + w.lrow, half, w.lhalf);
    }
  }
}

// Piece u of issue_step: u = 0..7 the operand row groups (even: Q group u/2,
// odd: P group u/2), u = 8 the scale dword.
template <int KIND, bool QNN = false>
__device__ __forceinline__ void issue_piece(int u, const OpStream& qst, const OpStream& pst, const ScaleSrc& sc,
                                            int64_t k, uint32_t dst, int wave) {
  using SM = Smem256<KIND>;
  constexpr int ES = KIND == GK_BF16 ? 2 : 1;
  constexpr int KSTEP = 128 / ES;
  const uint32_t kb = uint32_t(k * ES);
  v4i qrs;
  uint32_t kq;
  q_source<KIND, QNN>(qst, k, kb, qrs, kq);
  if (u < 8) {
    const int g = u >> 1;
    if ((u & 1) == 0) bdma16(qrs, qst.lane_off[g & 1], g * qst.group_bytes + kq, dst + (wave * 4 + g) * 1024);
    else bdma16(pst.rsrc, pst.lane_off[g & 1], g * pst.group_bytes + kb, dst + SM::kP + (wave * 4 + g) * 1024);
  } else if constexpr (KIND != GK_BF16) {
    bdma4(sc.rsrc, sc.voff, uint32_t((k / KSTEP) * sc.k), dst + sc.dst);
  }
}

// issue_step + read_half(st, 0, f) with the DMA instructions placed between
// the fragment reads (in the same order as the two functions), so the
// interleave puts them between the phase's MFMAs: issued as one burst after
// the barrier, a step's 72 DMA instructions per CU (~16 texture-address
// cycles each) held every wave back from its first MFMA.
template <int KIND, bool QNN = false>
__device__ __forceinline__ void issue_read_half0(const OpStream& qst, const OpStream& pst, const ScaleSrc& sc,
                                                 int64_t k, uint32_t dst, int wave, const uint8_t* st,
                                                 Frag<KIND>& f, const WaveCoord& w) {
  using SM = Smem256<KIND>;
  if constexpr (KIND == GK_BF16) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        if constexpr (QNN) f.a[s2][t] = read_frag16_nn(st, w.wi * 128 + t * 32, s2, w.lane);
        else f.a[s2][t] = read_frag16(st, w.wi * 128 + t * 32 + w.lrow, s2, w.lhalf);
        if (t < 2) f.b[s2][t] = read_frag16(st + SM::kP, w.wj * 64 + t * 32 + w.lrow, s2, w.lhalf);
      }
      issue_piece<KIND, QNN>(2 * t, qst, pst, sc, k, dst, wave);
      issue_piece<KIND, QNN>(2 * t + 1, qst, pst, sc, k, dst, wave);
    }
  } else {
    if constexpr (KIND == GK_FP8_MX) {
      const int blk = w.lhalf;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f.sa[t] = read_mx_scale(st, SM::kQS, w.wi * 128 + t * 32 + w.lrow, blk, w.q_mx_k);
        if (t < 2) f.sb[t] = read_mx_scale(st, SM::kPS, w.wj * 64 + t * 32 + w.lrow, blk, w.p_mx_k);
      }
    } else {
      f.sa[0] = read_pow2_scales(st, SM::kQS, w.wi * 128, w.lrow);
      const uint2 v = *reinterpret_cast<const uint2*>(
          st + SM::kPS + ((w.wj >> 1) * 128 + w.lrow * 4 + 2 * (w.wj & 1)) * 4);
      f.sb[0] = pack_exp4(v.x, v.y, 0u, 0u);
    }
    issue_piece<KIND, QNN>(8, qst, pst, sc, k, dst, wave);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if constexpr (QNN) f.a[t] = read_frag8_nn(st, w.wi * 128 + t * 32, 0, w.lane);
      else f.a[t] = read_frag8(st, w.wi * 128 + t * 32 + w.lrow, 0, w.lhalf);
      issue_piece<KIND, QNN>(2 * t, qst, pst, sc, k, dst, wave);
      if (t < 2) f.b[t] = read_frag8(st + SM::kP, w.wj * 64 + t * 32 + w.lrow, 0, w.lhalf);
      issue_piece<KIND, QNN>(2 * t + 1, qst, pst, sc, k, dst, wave);
    }
  }
}

template <int A, int B, int KIND>
__device__ __forceinline__ void mma_scaled(const Frag<KIND>& f, v16f (&acc)[4][2]) {
  acc[A][B] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.a[A], f.b[B], acc[A][B], 0, 0, A, f.sa[0], B,
                                                             f.sb[0]);
}

template <int KIND>
__device__ __forceinline__ void mma_half(const Frag<KIND>& f, v16f (&acc)[4][2]) {
  if constexpr (KIND == GK_BF16) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[s2][a], f.b[s2][b], acc[a][b], 0, 0, 0);
  } else if constexpr (KIND == GK_FP8_MX) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.a[a], f.b[b], acc[a][b], 0, 0, 0,
                                                                   f.sa[a], 0, f.sb[b]);
  } else {
    mma_scaled<0, 0>(f, acc);
    mma_scaled<0, 1>(f, acc);
    mma_scaled<1, 0>(f, acc);
    mma_scaled<1, 1>(f, acc);
    mma_scaled<2, 0>(f, acc);
    mma_scaled<2, 1>(f, acc);
    mma_scaled<3, 0>(f, acc);
    mma_scaled<3, 1>(f, acc);
  }
}

template <int KIND, bool QNN = false>
__device__ __forceinline__ void interleave_half() {
  constexpr int kMfma = KIND == GK_BF16 ? 16 : 8;
  // NN: four 8-byte reads per FP8 A fragment, two per BF16 one
  constexpr int kReads = KIND == GK_BF16 ? (QNN ? 2 : 1) : QNN ? 3 : 2;
#pragma unroll
  for (int i = 0; i < kMfma; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);  // LDS reads
  }
}

// A 256 x 256 workgroup tile: expert, first weight row i0, first token (or
// m) row j0, end of the valid j rows, and the contraction range.
struct Tile256 {
  int64_t e, i0, j0, j_end, k_lo, k_hi, slice;
};

// ragged-M: the valid 256-token tiles (sum over experts of ceil(rows / 256),
// from the device-side offsets; the launch is sized by a host bound) are
// split into 8 contiguous ranges, one per XCD (blockIdx % 8), for L2 reuse.
// ragged-K: when every expert runs and none holds more than 9/8 of the mean
// rows, the tiles are split into 8 contiguous ranges as well (each XCD then
// reads about one expert's operands); otherwise they stay in launch order, so
// one expert's tiles (whose K lengths differ between experts) spread over
// every XCD and the hardware's dynamic workgroup dispatch balances them.
// Returns false when this workgroup has no tile.
// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(v, d, 64);
    if (lane >= d) v += u;
  }
  return v;
}

template <int MODE>
__device__ __forceinline__ bool decode_tile256(const GemmParams& p, Tile256& t, int64_t bid) {
  const int64_t NI = (p.n_i + kT - 1) / kT;
  int64_t JT = 0, L;
  // Experts masked out (the other precision's launch) own no tiles here, so
  // the XCD ranges split only the work this launch does.
  auto unmasked = [&](int x) { return p.mask == nullptr || p.mask[x] == p.mask_want; };
  // ragged-M with at most 64 experts: lane x holds expert x's tile count, so
  // one wave-wide load of the offsets and a prefix scan replace the 2E
  // dependent loads of a serial walk (~6000 of a tile's ~60000 cycles at
  // 8 experts).
  const int lane = threadIdx.x & 63;
  const bool wide = MODE == GM_RAGGED_M && p.E <= 64;
  int cnt = 0, incl = 0, o0 = 0, o1 = 0;
  if (MODE == GM_RAGGED_M) {
    if (wide) {
      if (lane < p.E) {
        o0 = p.offsets[lane];
        o1 = p.offsets[lane + 1];
        if (unmasked(lane)) cnt = (o1 - o0 + kT - 1) / kT;
      }
      incl = wave_incl_scan(cnt, lane);
      JT = __builtin_amdgcn_readlane(incl, 63);
    } else {
      for (int x = 0; x < p.E; ++x)
        if (unmasked(x)) JT += (p.offsets[x + 1] - p.offsets[x] + kT - 1) / kT;
    }
    const int64_t n_valid = JT * NI;
    const int64_t per_xcd = (n_valid + 7) / 8;
    const int64_t k = bid / 8;
    if (k >= per_xcd) return false;
    L = (bid % 8) * per_xcd + k;
    if (L >= n_valid) return false;
  } else {
    L = bid;
    if ((p.rk_xcd & 1) && p.mask == nullptr && p.E <= 64) {
      int rows = lane < p.E ? p.offsets[lane + 1] - p.offsets[lane] : 0;
      int sum = rows, mx = rows;
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) {
        sum += __shfl_xor(sum, d, 64);
        mx = max(mx, __shfl_xor(mx, d, 64));
      }
      if (__builtin_amdgcn_readfirstlane(int(int64_t(mx) * p.E * 8 <= int64_t(sum) * 9))) {
        const int64_t per_xcd = (p.n_tiles + 7) / 8;
        L = (bid % 8) * per_xcd + bid / 8;
      }
    }
    if (L >= p.n_tiles) return false;
  }
  int64_t e = -1;
  if (MODE == GM_RAGGED_M) {
    const int64_t group = L / (kGroupM * NI);
    const int64_t first = group * kGroupM;
    const int64_t gsz = JT - first < kGroupM ? JT - first : kGroupM;
    const int64_t rem = L - group * kGroupM * NI;   // < gsz * NI
    int64_t J = first + (p.w_fast ? rem / NI : rem % gsz);
    t.i0 = (p.w_fast ? rem % NI : rem / gsz) * kT;
    // token tile J -> (expert, rows): an unmasked expert x holds
    // ceil(rows_x / 256) tiles
    if (wide) {
      const unsigned long long hit = __ballot(cnt > 0 && J >= incl - cnt && J < incl);
      if (hit == 0) return false;
      const int xe = __builtin_amdgcn_readfirstlane(__ffsll(hit) - 1);
      e = xe;
      t.j0 = int64_t(__builtin_amdgcn_readlane(o0, xe)) + (J - __builtin_amdgcn_readlane(incl - cnt, xe)) * kT;
      t.j_end = __builtin_amdgcn_readlane(o1, xe);
    } else {
      for (int x = 0; x < p.E; ++x) {
        const int64_t x0 = p.offsets[x], x1 = p.offsets[x + 1];
        const int64_t c = unmasked(x) ? (x1 - x0 + kT - 1) / kT : 0;
        if (J < c) {
          e = x;
          t.j0 = x0 + J * kT;
          t.j_end = x1;
          break;
        }
        J -= c;
      }
      if (e < 0) return false;
    }
    t.k_lo = 0;
    t.k_hi = p.K;
  } else {
    const int64_t NJ = (p.n_j + kT - 1) / kT;
    const int64_t per_e = NI * NJ;
    // split K: slice s of every tile follows all tiles of slice s - 1 (no
    // division on the unsplit path)
    t.slice = 0;
    if (p.splits > 1) {
      const int64_t per_slice = p.n_tiles / p.splits;
      t.slice = L / per_slice;
      L -= t.slice * per_slice;
    }
    e = L / per_e;
    const int64_t Lr = L % per_e;
    const int64_t group = Lr / (kGroupM * NJ);
    const int64_t first = group * kGroupM;
    const int64_t gsz = NI - first < kGroupM ? NI - first : kGroupM;
    const int64_t rem = Lr - group * kGroupM * NJ;   // < gsz * NJ
    t.i0 = (first + (p.rk_jfast ? rem / NJ : rem % gsz)) * kT;
    t.j0 = (p.rk_jfast ? rem % NJ : rem / gsz) * kT;
    t.j_end = p.n_j;
    // wave-uniform by construction; said so, the DMA takes them as scalars
    // also where the compiler cannot load them as such
    t.k_lo = __builtin_amdgcn_readfirstlane(p.offsets[e]);
    t.k_hi = __builtin_amdgcn_readfirstlane(p.offsets[e + 1]);
    if (p.splits > 1) {   // slice boundaries on the 128-row grid of the offsets
      const int64_t n = (t.k_hi - t.k_lo) / 128;
      t.k_hi = t.k_lo + 128 * (n * (t.slice + 1) / p.splits);
      t.k_lo += 128 * (n * t.slice / p.splits);
    }
  }
  if (p.mask != nullptr && p.mask[e] != p.mask_want) return false;
  t.e = e;
  return true;
}

// One 256 x 256 output tile of launch `p` (block index `bid` of that launch,
// two LDS stages at `smem`).  MXL (MX only): scale layouts, bit 0 = Q scales
// k-major, bit 1 = P scales k-major (row-major otherwise); fixed per
// instantiation so the unused address path costs no registers.
template <int KIND, int MODE, int MXL = 0>
__device__ __forceinline__ void gemm256_tile(const GemmParams& p, int64_t bid, uint8_t* smem) {
  using SM = Smem256<KIND>;
  constexpr int ES = KIND == GK_BF16 ? 2 : 1;         // element size
  constexpr int KSTEP = 128 / ES;                     // elements per 128-byte K step

  Tile256 tile;
  tile.slice = 0;
  if (!decode_tile256<MODE>(p, tile, bid)) return;
  const int64_t e = tile.e, i0 = tile.i0, j0 = tile.j0, j_end = tile.j_end, k_lo = tile.k_lo, k_hi = tile.k_hi;

  WaveCoord w;
  w.lane = threadIdx.x & 63;
  w.wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  w.wi = w.wave >> 2;   // wave tile: i [128*wi, +128), j [64*wj, +64)
  w.wj = w.wave & 3;
  w.lrow = w.lane & 31;
  w.lhalf = w.lane >> 5;
  w.q_mx_k = KIND == GK_FP8_MX && (MXL & 1) != 0;
  w.p_mx_k = KIND == GK_FP8_MX && (MXL & 2) != 0;
  const int64_t q_group = MODE == GM_RAGGED_M ? e : 0;
  // valid rows of each operand tile (multiples of 128)
  const int64_t q_rows = p.n_i - i0 < kT ? p.n_i - i0 : kT;
  const int64_t p_rows = j_end - j0 < kT ? j_end - j0 : kT;

  const OpStream qst = make_stream(p.Q.p + (q_group * p.Q.gs + i0 * p.Q.ld) * ES, p.Q.ld * ES, q_rows, w.lane,
                                   w.wave);
  const OpStream pst = make_stream(p.P.p + j0 * p.P.ld * ES, p.P.ld * ES, p_rows, w.lane, w.wave);

  // Scales: waves 0-3 fetch the Q scale slots, waves 4-7 the P slots, one
  // dword per lane per K step.
  ScaleSrc sc{};
  if constexpr (SM::kScaled) {
    const bool is_q = w.wave < 4;
    const int li = (w.wave & 3) * 64 + w.lane;   // slot 0..255
    sc = is_q ? make_scale_src<KIND>(p.Q, i0, q_rows, q_group, w.q_mx_k, li, SM::kQS)
              : make_scale_src<KIND>(p.P, j0, p_rows, 0, w.p_mx_k, li, SM::kPS);
  }

  v16f acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  // Two-stage pipeline, K step t in stage t % 2, fragments read one half-step
  // ahead into two register sets.  Iteration t (f0 holds half 0 of step t):
  //   A: MFMAs of (t, 0) while reading (t, 1) into f1;
  //   wait for this wave's DMA of step t+1 and its LDS reads, barrier (step
  //      t+1 has landed for every wave; no wave still reads stage t % 2);
  //   refill stage t % 2 with step t+2;
  //   B: MFMAs of (t, 1) while reading (t+1, 0) into f0.
  // No LDS read waits behind a barrier with the matrix pipe idle.  The refills
  // are unconditional (clamped to the last step), which keeps the loop body
  // one basic block; the reads after the last step re-read a valid stage.
  const int64_t nk = (k_hi - k_lo) / KSTEP;
  if (nk > 0) {
    const uint32_t smem_lds = lds_addr(smem);
    Frag<KIND> f0, f1;
    issue_step<KIND>(qst, pst, sc, k_lo, smem_lds, w.wave);
    issue_step<KIND>(qst, pst, sc, k_lo + (nk > 1 ? KSTEP : 0), smem_lds + SM::kStage, w.wave);
    // step 0 has landed once at most step 1's DMAs are still in flight
    FM_WAIT_VMCNT(KIND == GK_BF16 ? 8 : 9);
    block_barrier();
    read_half<KIND>(smem, 0, f0, w);
    int cur_off = 0;
#pragma unroll 1
    for (int64_t t = 0; t < nk; ++t) {
      const int nxt_off = SM::kStage - cur_off;
      __builtin_amdgcn_sched_barrier(0);
      read_half<KIND>(smem + cur_off, 1, f1, w);
      if constexpr (KIND == GK_FP8_POW2) {
        f1.sa[0] = f0.sa[0];
        f1.sb[0] = f0.sb[0];
      }
      mma_half<KIND>(f0, acc);
      interleave_half<KIND>();
      __builtin_amdgcn_sched_barrier(0);
      FM_WAIT_VMCNT(0);
      block_barrier();
      const int64_t t2n = t + 2 < nk ? t + 2 : nk - 1;
      issue_read_half0<KIND>(qst, pst, sc, k_lo + t2n * KSTEP, smem_lds + cur_off, w.wave, smem + nxt_off, f0, w);
      mma_half<KIND>(f1, acc);
      interleave_half<KIND>();
      __builtin_amdgcn_sched_barrier(0);
      cur_off = nxt_off;
    }
    FM_WAIT_VMCNT(0);  // no LDS-DMA may still be in flight when the workgroup exits
  }

  // -------------------------------------------------------------- epilogue ----
  // The output row is j (a token in ragged-M, an m row of the weight gradient
  // in ragged-K, whose operands the launcher swapped) and the contiguous
  // column is i, so each lane holds 4 consecutive columns of one row.  n_i,
  // the valid rows and split are multiples of 128: every bound below holds or
  // fails for a wave's whole 128 x 64 block.
  const int wi = w.wi, wj = w.wj, lrow = w.lrow, lhalf = w.lhalf, lane = w.lane;
  const int64_t ib = i0 + wi * 128, jb = j0 + wj * 64;
  const bool live = ib < p.n_i && jb < j0 + p_rows;
  int64_t row_off;
  void* C;
  if (MODE == GM_RAGGED_M) {
    C = p.C;
    row_off = jb * p.ldC + ib;
  } else {
    const bool second = uniform_ge(jb, p.split);
    C = second ? p.C2 : p.C;
    row_off = e * (second ? p.c2_gs : p.c_gs) + (second ? jb - p.split : jb) * p.ldC + ib + tile.slice * p.ws_slice;
  }
  if (!p.out_f32) {
    // bf16: each wave stages its 64 x 128 block in its own 16 KiB of LDS and
    // writes it back as whole 256-byte row segments (after a barrier: every
    // DMA has landed and every read of the stages is done).
    block_barrier();
    if (!live) return;
    uint8_t* W = smem + w.wave * 16384;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int jr = b * 32 + lrow;
          uint2 v;
          v.x = hw_bf16x2(acc[a][b][4 * q], acc[a][b][4 * q + 1]);
          v.y = hw_bf16x2(acc[a][b][4 * q + 2], acc[a][b][4 * q + 3]);
          *reinterpret_cast<uint2*>(W + jr * 256 + (((a * 4 + q) ^ (jr & 15)) << 4) + lhalf * 8) = v;
        }
    const int c = lane & 15;
    uint16_t* dst = static_cast<uint16_t*>(C) + row_off + c * 8;
    if ((p.ldC & 7) == 0) {   // whole 16-byte stores; the split form in a loop of its own
#pragma unroll 4
      for (int n = 0; n < 16; ++n) {
        const int rr = n * 4 + (lane >> 4);
        const uint4 v = *reinterpret_cast<const uint4*>(W + rr * 256 + ((c ^ (rr & 15)) << 4));
        st_global(dst + rr * p.ldC, v);
      }
    } else {
#pragma unroll 4
      for (int n = 0; n < 16; ++n) {
        const int rr = n * 4 + (lane >> 4);
        const uint4 v = *reinterpret_cast<const uint4*>(W + rr * 256 + ((c ^ (rr & 15)) << 4));
        uint2* d = reinterpret_cast<uint2*>(dst + rr * p.ldC);
        st_global(d, make_uint2(v.x, v.y));
        st_global(d + 1, make_uint2(v.z, v.w));
      }
    }
    return;
  }
  if (!live) return;
  float* dst = static_cast<float*>(C) + row_off + lrow * p.ldC + 4 * lhalf;
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        st_global(dst + b * 32 * p.ldC + a * 32 + 8 * q,
            make_float4(acc[a][b][4 * q], acc[a][b][4 * q + 1], acc[a][b][4 * q + 2], acc[a][b][4 * q + 3]));
}

template <int KIND, int MODE, int MXL = 0>
__global__ __launch_bounds__(512) void gemm256_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * Smem256<KIND>::kStage];
  gemm256_tile<KIND, MODE, MXL>(p, blockIdx.x, smem);
}

// A ragged-M launch (blocks [0, nbm), nbm a multiple of 8 so both keep their
// XCD mapping) and a ragged-K launch (the blocks after it) as one grid: the
// dgrad dH = dY w2 and the weight gradient dW2 read the same permuted dY and
// are independent, and run back to back each leaves its last round of tiles
// part-empty (1.5 rounds each at configs[2]'s shapes; 3 rounds together).
template <int KIND>
__global__ __launch_bounds__(512) void gemm256_mk_kernel(GemmParams pm, GemmParams pk, int64_t nbm) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * Smem256<KIND>::kStage];
  const int64_t b = blockIdx.x;
  if (b < nbm) gemm256_tile<KIND, GM_RAGGED_M>(pm, b, smem);
  else gemm256_tile<KIND, GM_RAGGED_K>(pk, b - nbm, smem);
}

// ============================================================================
// Persistent ragged-M variant of the 256 x 256 kernel
// ============================================================================
// One workgroup per CU walks a strided share of its XCD's contiguous tile
// range (the same XCD split and L2 grouping as decode_tile256).  The last two
// refills of a tile's K loop fetch the next tile's first two K steps instead
// of clamped duplicates, and the bf16 epilogue stages through LDS beyond the
// two operand stages (2 KiB per wave), so a tile's output stores, the next
// tile's first loads and its decode (registers only: the per-expert tile
// counts are read once per workgroup) overlap.  Needs at most 64 experts and
// at least two K steps (the launcher falls back to gemm256_kernel otherwise).
// Per-lane values (expert x = lane: tile count, inclusive scan, offsets) live
// in the wave's own 1 KiB of LDS between tiles, so they cost no registers
// across the K loop.
// The lane id read from the hardware (v_mbcnt) at each use.  Volatile, so the
// compiler neither hoists nor shares it: values derived from the lane between
// tiles are rebuilt from it instead of being kept live across the K loops,
// where the register budget is spent (a spilled value's reload waits for
// every load in flight, the operand prefetch included).
__device__ __forceinline__ int fresh_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

struct TileQueue {
  int* lds;                    // [4][64] ints of this wave
  int NI, JT, n_valid, per_xcd, xcd, c0, nbx, w_fast;
};

// A tile of the persistent kernel: expert, first weight row, first token row,
// end of the expert's rows (32-bit: the padded buffer has int32 offsets).
struct TileP {
  int e, i0, j0, j_end;
};

// Every wave computes the same values; wave 0 writes the one LDS copy, which
// the others read after the barrier that follows.
__device__ __forceinline__ void tile_queue_init(const GemmParams& p, TileQueue& q, int* lds) {
  const int lane = threadIdx.x & 63;
  int cnt = 0, o0 = 0, o1 = 0;
  if (lane < p.E) {
    o0 = p.offsets[lane];
    o1 = p.offsets[lane + 1];
    if (p.mask == nullptr || p.mask[lane] == p.mask_want) cnt = (o1 - o0 + kT - 1) / kT;
  }
  const int incl = wave_incl_scan(cnt, lane);
  q.lds = lds;
  if (threadIdx.x < 64) {
    lds[lane] = cnt;
    lds[64 + lane] = incl;
    lds[128 + lane] = o0;
    lds[192 + lane] = o1;
  }
  q.NI = int((p.n_i + kT - 1) / kT);
  q.JT = __builtin_amdgcn_readlane(incl, 63);
  q.n_valid = q.JT * q.NI;
  q.per_xcd = (q.n_valid + 7) / 8;
  q.xcd = int(blockIdx.x % 8);
  q.c0 = int(blockIdx.x / 8);
  q.nbx = int(gridDim.x / 8);
  q.w_fast = p.w_fast;
}

// The m-th tile of this workgroup, false past the end of its share.
__device__ __forceinline__ bool tile_queue_get(const TileQueue& q, int m, TileP& t) {
  const int loc = q.c0 + m * q.nbx;
  if (loc >= q.per_xcd) return false;
  const int L = q.xcd * q.per_xcd + loc;
  if (L >= q.n_valid) return false;
  const int group = L / (kGroupM * q.NI);
  const int first = group * kGroupM;
  const int gsz = q.JT - first < kGroupM ? q.JT - first : kGroupM;
  const int rem = L - group * kGroupM * q.NI;   // < gsz * NI
  const int J = first + (q.w_fast ? rem / q.NI : rem % gsz);
  t.i0 = (q.w_fast ? rem % q.NI : rem / gsz) * kT;
  const int lane = fresh_lane();
  const int cnt = q.lds[lane], incl = q.lds[64 + lane];
  const unsigned long long hit = __ballot(cnt > 0 && J >= incl - cnt && J < incl);
  if (hit == 0) return false;
  const int xe = __builtin_amdgcn_readfirstlane(__ffsll(hit) - 1);
  t.e = xe;
  t.j0 = q.lds[128 + xe] + (J - (q.lds[64 + xe] - q.lds[xe])) * kT;
  t.j_end = q.lds[192 + xe];
  return true;
}

// DMA sources of one tile.
struct TileStreams {
  OpStream q, p;
  ScaleSrc sc;
};

template <int KIND, bool QNN = false>
__device__ __forceinline__ TileStreams tile_streams(const Operand& Q, const Operand& P, int64_t n_i, const TileP& t,
                                                   const WaveCoord& w) {
  using SM = Smem256<KIND>;
  constexpr int ES = KIND == GK_BF16 ? 2 : 1;
  TileStreams s;
  const int64_t q_rows = n_i - t.i0 < kT ? n_i - t.i0 : kT;
  const int64_t p_rows = t.j_end - t.j0 < kT ? t.j_end - t.j0 : kT;
  const int lane = fresh_lane();
  if constexpr (QNN) {
    if constexpr (KIND == GK_BF16) {   // a split operand splits along K here
      const int64_t off = (int64_t(t.e) * Q.gs + int64_t(t.i0)) * 2;
      s.q = make_stream_nn16(Q.p + off, Q.p2 + off, Q.split, Q.ld * 2, lane, w.wave);
    } else {
      s.q = make_stream_nn(Q.p + int64_t(t.e) * Q.gs + int64_t(t.i0), Q.ld, lane, w.wave);
    }
  } else {   // a tile lies in one of the two tensors of a split operand (split % 256 == 0)
    const bool second = t.i0 >= Q.split;
    const int64_t qi = second ? t.i0 - Q.split : t.i0;
    s.q = make_stream((second ? Q.p2 : Q.p) + (int64_t(t.e) * Q.gs + qi * Q.ld) * ES, Q.ld * ES, q_rows, lane,
                      w.wave);
  }
  s.p = make_stream(P.p + int64_t(t.j0) * P.ld * ES, P.ld * ES, p_rows, lane, w.wave);
  s.sc = ScaleSrc{};
  if constexpr (SM::kScaled) {
    const int li = (w.wave & 3) * 64 + lane;
    s.sc = w.wave < 4 ? make_scale_src<KIND>(Q, t.i0, q_rows, t.e, w.q_mx_k, li, SM::kQS)
                      : make_scale_src<KIND>(P, t.j0, p_rows, 0, w.p_mx_k, li, SM::kPS);
  }
  return s;
}

// Kernel-argument fields read back from the workgroup's LDS copy as
// wave-uniform (scalar) values.
__device__ __forceinline__ int64_t rfl64(int64_t v) {
  const uint64_t u = uint64_t(v);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(u));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(u >> 32));
  return int64_t((uint64_t(hi) << 32) | lo);
}
__device__ __forceinline__ Operand uniform_operand(const Operand* o) {
  Operand r;
  r.p = reinterpret_cast<const uint8_t*>(rfl64(int64_t(size_t(o->p))));
  r.ld = rfl64(o->ld);
  r.gs = rfl64(o->gs);
  r.s = reinterpret_cast<const void*>(rfl64(int64_t(size_t(o->s))));
  r.s_row = rfl64(o->s_row);
  r.s_kb = rfl64(o->s_kb);
  r.s_gs = rfl64(o->s_gs);
  r.s_shift = __builtin_amdgcn_readfirstlane(o->s_shift);
  r.p2 = reinterpret_cast<const uint8_t*>(rfl64(int64_t(size_t(o->p2))));
  r.split = rfl64(o->split);
  return r;
}

// bf16 epilogue of one wave's 128 (i) x 64 (j) block through its own 2 KiB
// of LDS `W`: 8 passes of 32 rows x 32 columns (block b of the rows, block a
// of the columns), each written back as 64-byte row segments.  16-byte chunk
// q of row r sits at position q ^ ((r / 4) % 4).
// VEC16: whole 16-byte stores (ldC a multiple of 8), chosen once per call so
// that the two store forms stay separate instructions.
template <bool VEC16>
__device__ __forceinline__ void store_bf16_passes_v(const v16f (&acc)[4][2], uint8_t* W, uint16_t* C, int64_t ldC,
                                                    int64_t row0, int64_t col0, const WaveCoord& w) {
  const int lrow = w.lrow, lhalf = w.lhalf, lane = w.lane;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int a = 0; a < 4; ++a) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint2 v;
        v.x = hw_bf16x2(acc[a][b][4 * q], acc[a][b][4 * q + 1]);
        v.y = hw_bf16x2(acc[a][b][4 * q + 2], acc[a][b][4 * q + 3]);
        *reinterpret_cast<uint2*>(W + lrow * 64 + ((q ^ ((lrow >> 2) & 3)) << 4) + lhalf * 8) = v;
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int r = u * 16 + (lane >> 2), c = lane & 3;
        const uint4 v = *reinterpret_cast<const uint4*>(W + r * 64 + ((c ^ ((r >> 2) & 3)) << 4));
        uint16_t* d = C + (row0 + b * 32 + r) * ldC + col0 + a * 32 + c * 8;
        if constexpr (VEC16) {
          st_global(d, v);
        } else {
          st_global(d, make_uint2(v.x, v.y));
          st_global(d + 4, make_uint2(v.z, v.w));
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
}

__device__ __forceinline__ void store_bf16_passes(const v16f (&acc)[4][2], uint8_t* W, uint16_t* C, int64_t ldC,
                                                  int64_t row0, int64_t col0, const WaveCoord& w) {
  if ((ldC & 7) == 0) store_bf16_passes_v<true>(acc, W, C, ldC, row0, col0, w);
  else store_bf16_passes_v<false>(acc, W, C, ldC, row0, col0, w);
}

// QNN (BF16 and FP8 pow2): the weight operand Q is stored [K][N]
// (make_stream_nn16 / read_frag16_nn, make_stream_nn / read_frag8_nn); all N
// tiles are full (N % 256 == 0, checked by the launcher).
template <int KIND, int MXL = 0, bool QNN = false>
__global__ __launch_bounds__(512) void gemm256p_kernel(GemmParams p) {
  using SM = Smem256<KIND>;
  constexpr int ES = KIND == GK_BF16 ? 2 : 1;
  constexpr int KSTEP = 128 / ES;
  constexpr int kSpare = 8 * 2048;   // epilogue staging, 2 KiB per wave
  constexpr int kQueue = 1024;       // tile queue
  constexpr int kArgs = (sizeof(GemmParams) + 15) / 16 * 16;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * SM::kStage + kSpare + kQueue + kArgs];
  // The operand descriptors are needed once per tile; the workgroup's LDS copy
  // keeps them out of the scalar registers across the K loop.
  GemmParams* const pl = reinterpret_cast<GemmParams*>(smem + 2 * SM::kStage + kSpare + kQueue);
  if (threadIdx.x == 0) *pl = p;   // read only after the prologue barrier

  WaveCoord w;
  w.lane = threadIdx.x & 63;
  w.wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  w.wi = w.wave >> 2;
  w.wj = w.wave & 3;
  w.lrow = w.lane & 31;
  w.lhalf = w.lane >> 5;
  w.q_mx_k = KIND == GK_FP8_MX && (MXL & 1) != 0;
  w.p_mx_k = KIND == GK_FP8_MX && (MXL & 2) != 0;

  TileQueue tq;
  tile_queue_init(p, tq, reinterpret_cast<int*>(smem + 2 * SM::kStage + kSpare));
  block_barrier();   // the tile queue is in LDS
  TileP cur;
  if (!tile_queue_get(tq, 0, cur)) return;
  TileStreams S = tile_streams<KIND, QNN>(p.Q, p.P, p.n_i, cur, w);
  const int64_t nk = p.K / KSTEP;   // >= 2 (launcher)
  const uint32_t smem_lds = lds_addr(smem);
  uint8_t* const W = smem + 2 * SM::kStage + w.wave * 2048;

  Frag<KIND> f0, f1;
  issue_step<KIND, QNN>(S.q, S.p, S.sc, 0, smem_lds, w.wave);
  issue_step<KIND, QNN>(S.q, S.p, S.sc, KSTEP, smem_lds + SM::kStage, w.wave);
  FM_WAIT_VMCNT(KIND == GK_BF16 ? 8 : 9);
  block_barrier();
  read_half<KIND, QNN>(smem, 0, f0, w);
  int cur_off = 0;

  for (int m = 0;; ++m) {
    TileP nxt;
    const bool has_next = tile_queue_get(tq, m + 1, nxt);
    v16f acc[4][2];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

    // The loop of gemm256_kernel, as two branch-free loops (one basic block
    // each, so the MFMA / LDS-read interleave and the explicit vmcnt waits hold):
    // steps 0 .. nk-3 refill this tile's steps t+2; the last two refill the
    // next tile's steps 0 and 1 (duplicates of the last step on the last tile).
    auto step = [&](int64_t t, int64_t kn) {
      const int nxt_off = SM::kStage - cur_off;
      __builtin_amdgcn_sched_barrier(0);
      read_half<KIND, QNN>(smem + cur_off, 1, f1, w);
      if constexpr (KIND == GK_FP8_POW2) {
        f1.sa[0] = f0.sa[0];
        f1.sb[0] = f0.sb[0];
      }
      mma_half<KIND>(f0, acc);
      interleave_half<KIND, QNN>();
      __builtin_amdgcn_sched_barrier(0);
      FM_WAIT_VMCNT(0);
      block_barrier();
      issue_read_half0<KIND, QNN>(S.q, S.p, S.sc, kn * KSTEP, smem_lds + cur_off, w.wave, smem + nxt_off, f0, w);
      mma_half<KIND>(f1, acc);
      interleave_half<KIND, QNN>();
      __builtin_amdgcn_sched_barrier(0);
      cur_off = nxt_off;
    };
#pragma unroll 1
    for (int64_t t = 0; t < nk - 2; ++t) step(t, t + 2);
    // this tile's sources are dead now: S becomes the next tile's
    if (has_next) {
      const Operand Q = uniform_operand(&pl->Q), P = uniform_operand(&pl->P);
      S = tile_streams<KIND, QNN>(Q, P, rfl64(pl->n_i), nxt, w);
    }
#pragma unroll 1
    for (int64_t t = nk - 2; t < nk; ++t) step(t, has_next ? t + 2 - nk : nk - 1);

    // epilogue of `cur` (output row j = token, contiguous column i)
    const int64_t ib = cur.i0 + w.wi * 128, jb = cur.j0 + w.wj * 64;
    const int p_rows = cur.j_end - cur.j0 < kT ? cur.j_end - cur.j0 : kT;
    if (ib < p.n_i && jb < cur.j0 + p_rows) {
      WaveCoord we = w;
      we.lane = fresh_lane();
      we.lrow = we.lane & 31;
      we.lhalf = we.lane >> 5;
      if (!p.out_f32) {
        store_bf16_passes(acc, W, static_cast<uint16_t*>(p.C), p.ldC, jb, ib, we);
      } else {
        float* dst = static_cast<float*>(p.C) + jb * p.ldC + ib + we.lrow * p.ldC + 4 * we.lhalf;
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              st_global(dst + b * 32 * p.ldC + a * 32 + 8 * q, make_float4(
                  acc[a][b][4 * q], acc[a][b][4 * q + 1], acc[a][b][4 * q + 2], acc[a][b][4 * q + 3]));
      }
    }
    if (!has_next) break;
    cur = nxt;
  }
  FM_WAIT_VMCNT(0);  // no LDS-DMA may still be in flight when the workgroup exits
}

// ============================================================================
// Persistent ragged-K variant (weight gradients)
// ============================================================================
// gemm256p_kernel's loop over ragged-K tiles: expert e's output tiles (i: b_t
// rows, j: a_t rows) contract over its token range [offsets[e], offsets[e+1]),
// so each tile has its own K range, and the last two refills of a tile fetch
// the next tile's first two K steps.  That pipeline needs at least two K steps
// per tile: tiles of experts with fewer rows ("short": zero or one K step) are
// skipped by the pipelined walk and done afterwards one at a time.  No expert
// mask, no K split, at most 64 experts (checked by the launcher).  Each
// workgroup walks a share of the tiles: one of 8 contiguous per-XCD ranges
// when the experts are balanced (as decode_tile256), otherwise the tiles a
// one-tile-per-block launch would give blocks b, b + G, b + 2 G, ... (G the
// grid), so the tiles running at once are neighbours sharing operands.
struct TileK {
  int e, i0, j0, k_lo, nk;
};

struct RkQueue {
  const int* off;   // LDS copy of offsets[0 .. E]
  int NI, NJ, per_e, n_tiles, per_xcd, xcd, c0, nbx, contiguous, chunked, jfast;
};

// The c-th tile of this workgroup's share, false past its end.  Shares:
// contiguous -- XCD x walks the x-th of 8 contiguous tile ranges;
// chunked    -- round c of XCD x is the chunk of nbx consecutive tiles
//               (8 c + x) nbx .. +nbx, so the tiles an XCD runs at once are
//               neighbours sharing operand rows (L2 reuse) while every XCD
//               still takes an equal share of every expert's tiles;
// otherwise  -- the tiles a one-tile-per-block launch gives block xcd + 8 loc.
__device__ __forceinline__ bool rk_tile_at(const RkQueue& q, int c, TileK& t, int kstep) {
  const int loc = q.c0 + c * q.nbx;
  int L;
  if (q.contiguous) {
    if (loc >= q.per_xcd) return false;
    L = q.xcd * q.per_xcd + loc;
  } else if (q.chunked) {
    L = (c * 8 + q.xcd) * q.nbx + q.c0;
  } else {
    L = q.xcd + 8 * loc;   // block index xcd + 8 loc of a one-tile-per-block launch
  }
  if (L >= q.n_tiles) return false;
  const int e = L / q.per_e, Lr = L - e * q.per_e;
  const int group = Lr / (kGroupM * q.NJ);
  const int first = group * kGroupM;
  const int gsz = q.NI - first < kGroupM ? q.NI - first : kGroupM;
  const int rem = Lr - group * kGroupM * q.NJ;   // < gsz * NJ
  t.e = e;
  t.i0 = (first + (q.jfast ? rem / q.NJ : rem % gsz)) * kT;
  t.j0 = (q.jfast ? rem % q.NJ : rem / gsz) * kT;
  t.k_lo = __builtin_amdgcn_readfirstlane(q.off[e]);   // wave-uniform: it feeds the DMA's scalar offset
  t.nk = (__builtin_amdgcn_readfirstlane(q.off[e + 1]) - t.k_lo) / kstep;
  return true;
}

// The next tile of the share with at least two K steps, from position `c`.
__device__ __forceinline__ bool rk_next_long(const RkQueue& q, int& c, TileK& t, int kstep) {
  for (;;) {
    if (!rk_tile_at(q, c, t, kstep)) return false;
    ++c;
    if (t.nk >= 2) return true;
  }
}

template <int KIND, int MXL = 0>
__global__ __launch_bounds__(512) void gemm256pk_kernel(GemmParams p) {
  using SM = Smem256<KIND>;
  constexpr int ES = KIND == GK_BF16 ? 2 : 1;
  constexpr int KSTEP = 128 / ES;
  constexpr int kSpare = 8 * 2048;   // epilogue staging, 2 KiB per wave
  constexpr int kQueue = 1024;       // offsets copy
  constexpr int kArgs = (sizeof(GemmParams) + 15) / 16 * 16;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * SM::kStage + kSpare + kQueue + kArgs];
  GemmParams* const pl = reinterpret_cast<GemmParams*>(smem + 2 * SM::kStage + kSpare + kQueue);
  int* const off = reinterpret_cast<int*>(smem + 2 * SM::kStage + kSpare);
  if (threadIdx.x == 0) *pl = p;   // read only after the first barrier

  // the offsets into LDS; the expert balance for the XCD split
  const int lane0 = threadIdx.x & 63;
  int rows = 0, o0 = 0;
  if (lane0 < p.E) {
    o0 = p.offsets[lane0];
    rows = p.offsets[lane0 + 1] - o0;
  }
  if (threadIdx.x < 64) {
    if (lane0 < p.E) off[lane0] = o0;
    if (lane0 == p.E - 1) off[p.E] = o0 + rows;
  }
  int sum = rows, mx = rows;
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    sum += __shfl_xor(sum, d, 64);
    mx = max(mx, __shfl_xor(mx, d, 64));
  }
  block_barrier();   // offsets and arguments are in LDS

  WaveCoord w;
  w.lane = threadIdx.x & 63;
  w.wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  w.wi = w.wave >> 2;
  w.wj = w.wave & 3;
  w.lrow = w.lane & 31;
  w.lhalf = w.lane >> 5;
  w.q_mx_k = KIND == GK_FP8_MX && (MXL & 1) != 0;
  w.p_mx_k = KIND == GK_FP8_MX && (MXL & 2) != 0;

  RkQueue q;
  q.off = off;
  q.NI = int((p.n_i + kT - 1) / kT);
  q.NJ = int((p.n_j + kT - 1) / kT);
  q.per_e = q.NI * q.NJ;
  q.n_tiles = int(p.n_tiles);
  // wave-uniform (the shuffles leave every lane the same values, which the
  // compiler cannot see): the tile walk feeds the DMA's scalar offsets
  q.contiguous = __builtin_amdgcn_readfirstlane(int((p.rk_xcd & 1) && int64_t(mx) * p.E * 8 <= int64_t(sum) * 9));
  q.chunked = !q.contiguous && (p.rk_xcd & 2) != 0;
  q.per_xcd = (q.n_tiles + 7) / 8;
  q.xcd = int(blockIdx.x % 8);
  q.c0 = int(blockIdx.x / 8);
  q.nbx = int(gridDim.x / 8);
  q.jfast = p.rk_jfast;
  auto streams = [&](const TileK& t) {
    const Operand Q = uniform_operand(&pl->Q), P = uniform_operand(&pl->P);
    return tile_streams<KIND>(Q, P, rfl64(pl->n_i), TileP{0, t.i0, t.j0, int(rfl64(pl->n_j))}, w);
  };
  const uint32_t smem_lds = lds_addr(smem);
  uint8_t* const W = smem + 2 * SM::kStage + w.wave * 2048;

  // output row j (an a_t row: m of the weight gradient), contiguous column i;
  // rows at or past `split` go to C2
  auto epilogue = [&](const TileK& t, const v16f (&acc)[4][2]) {
    const int64_t n_i = rfl64(pl->n_i), n_j = rfl64(pl->n_j);
    const int64_t ib = t.i0 + w.wi * 128, jb = t.j0 + w.wj * 64;
    if (ib >= n_i || jb >= n_j) return;
    const int64_t split = rfl64(pl->split);
    const bool second = uniform_ge(jb, split);
    void* const Cb = second ? pl->C2 : pl->C;
    const int64_t gs = second ? rfl64(pl->c2_gs) : rfl64(pl->c_gs);
    const int64_t ldC = rfl64(pl->ldC);
    const int64_t row0 = second ? jb - split : jb;
    WaveCoord we = w;
    we.lane = fresh_lane();
    we.lrow = we.lane & 31;
    we.lhalf = we.lane >> 5;
    if (!p.out_f32) {
      store_bf16_passes(acc, W, static_cast<uint16_t*>(Cb) + int64_t(t.e) * gs, ldC, row0, ib, we);
    } else {
      float* dst = static_cast<float*>(Cb) + int64_t(t.e) * gs + row0 * ldC + ib + we.lrow * ldC + 4 * we.lhalf;
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4)
            st_global(dst + b * 32 * ldC + a * 32 + 8 * r4, make_float4(
                acc[a][b][4 * r4], acc[a][b][4 * r4 + 1], acc[a][b][4 * r4 + 2], acc[a][b][4 * r4 + 3]));
    }
  };

  Frag<KIND> f0, f1;
  int cursor = 0;
  TileK cur;
  if (rk_next_long(q, cursor, cur, KSTEP)) {
    TileStreams S = streams(cur);
    issue_step<KIND>(S.q, S.p, S.sc, cur.k_lo, smem_lds, w.wave);
    issue_step<KIND>(S.q, S.p, S.sc, cur.k_lo + KSTEP, smem_lds + SM::kStage, w.wave);
    FM_WAIT_VMCNT(KIND == GK_BF16 ? 8 : 9);
    block_barrier();
    read_half<KIND>(smem, 0, f0, w);
    int cur_off = 0;
    for (;;) {
      TileK nxt;
      const bool has_next = rk_next_long(q, cursor, nxt, KSTEP);
      v16f acc[4][2];
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

      // as gemm256p_kernel: steps 0 .. nk-3 refill this tile's steps t+2, the
      // last two the next tile's steps 0 and 1 (this tile's last step again on
      // the last tile); `k` is the absolute contraction offset of the refill
      auto step = [&](int64_t k) {
        const int nxt_off = SM::kStage - cur_off;
        __builtin_amdgcn_sched_barrier(0);
        read_half<KIND>(smem + cur_off, 1, f1, w);
        if constexpr (KIND == GK_FP8_POW2) {
          f1.sa[0] = f0.sa[0];
          f1.sb[0] = f0.sb[0];
        }
        mma_half<KIND>(f0, acc);
        interleave_half<KIND>();
        __builtin_amdgcn_sched_barrier(0);
        FM_WAIT_VMCNT(0);
        block_barrier();
        issue_read_half0<KIND>(S.q, S.p, S.sc, k, smem_lds + cur_off, w.wave, smem + nxt_off, f0, w);
        mma_half<KIND>(f1, acc);
        interleave_half<KIND>();
        __builtin_amdgcn_sched_barrier(0);
        cur_off = nxt_off;
      };
      const int nk = cur.nk;   // >= 2
#pragma unroll 1
      for (int t = 0; t < nk - 2; ++t) step(int64_t(cur.k_lo) + int64_t(t + 2) * KSTEP);
      const int64_t last = int64_t(cur.k_lo) + int64_t(nk - 1) * KSTEP;
      if (has_next) S = streams(nxt);
#pragma unroll 1
      for (int t = 0; t < 2; ++t) step(has_next ? int64_t(nxt.k_lo) + int64_t(t) * KSTEP : last);
      epilogue(cur, acc);
      if (!has_next) break;
      cur = nxt;
    }
    FM_WAIT_VMCNT(0);
    block_barrier();   // the stages are free again
  }

  // short tiles of the share: zero or one K step each
  for (int c = 0;; ++c) {
    TileK t;
    if (!rk_tile_at(q, c, t, KSTEP)) break;
    if (t.nk >= 2) continue;
    v16f acc[4][2];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;
    if (t.nk == 1) {
      const TileStreams S = streams(t);
      issue_step<KIND>(S.q, S.p, S.sc, t.k_lo, smem_lds, w.wave);
      FM_WAIT_VMCNT(0);
      block_barrier();
      read_half<KIND>(smem, 0, f0, w);
      read_half<KIND>(smem, 1, f1, w);
      if constexpr (KIND == GK_FP8_POW2) {
        f1.sa[0] = f0.sa[0];
        f1.sb[0] = f0.sb[0];
      }
      mma_half<KIND>(f0, acc);
      mma_half<KIND>(f1, acc);
      block_barrier();   // every wave has read the stage before the next tile's DMA
    }
    epilogue(t, acc);
  }
}

// ============================================================================
// Persistent dgrad + weight-gradient grid (fm_grouped_gemm_ragged_m_k)
// ============================================================================
// gemm256_mk_kernel's pair of launches walked by one persistent pipeline:
// each workgroup takes its share of the ragged-M tiles (the per-XCD ranges of
// gemm256p_kernel), then its share of the ragged-K tiles (those of
// gemm256pk_kernel, the workgroups of an XCD in reverse order, so the ones
// with an extra ragged-M tile get one fewer ragged-K tile), and the refills
// of a tile's last two K steps fetch the next tile's first two whichever
// launch it belongs to.  Ragged-K tiles of fewer than two K steps come last,
// one at a time.  No expert masks, at most 64 experts, at least two ragged-M
// K steps (checked by the launcher).
struct ItemMK {
  int k_mode;   // 0: a ragged-M tile (pm), 1: a ragged-K tile (pk)
  int e, i0, j0, j_end, k_base, nk;
};

template <int KIND>
__global__ __launch_bounds__(512) void gemm256pmk_kernel(GemmParams pm, GemmParams pk) {
  using SM = Smem256<KIND>;
  constexpr int ES = KIND == GK_BF16 ? 2 : 1;
  constexpr int KSTEP = 128 / ES;
  constexpr int kSpare = 8 * 2048;   // epilogue staging, 2 KiB per wave
  constexpr int kQueue = 1024;       // ragged-M tile queue
  constexpr int kOff = 512;          // ragged-K offsets copy
  constexpr int kArgs = (sizeof(GemmParams) + 15) / 16 * 16;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * SM::kStage + kSpare + kQueue + kOff + 2 * kArgs];
  int* const qlds = reinterpret_cast<int*>(smem + 2 * SM::kStage + kSpare);
  int* const off = reinterpret_cast<int*>(smem + 2 * SM::kStage + kSpare + kQueue);
  GemmParams* const plm = reinterpret_cast<GemmParams*>(smem + 2 * SM::kStage + kSpare + kQueue + kOff);
  GemmParams* const plk = reinterpret_cast<GemmParams*>(smem + 2 * SM::kStage + kSpare + kQueue + kOff + kArgs);
  if (threadIdx.x == 0) {
    *plm = pm;
    *plk = pk;
  }

  WaveCoord w;
  w.lane = threadIdx.x & 63;
  w.wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  w.wi = w.wave >> 2;
  w.wj = w.wave & 3;
  w.lrow = w.lane & 31;
  w.lhalf = w.lane >> 5;
  w.q_mx_k = false;
  w.p_mx_k = false;

  // ragged-M queue (LDS) and the ragged-K offsets (LDS); balance of the experts
  TileQueue tq;
  tile_queue_init(pm, tq, qlds);
  const int lane0 = threadIdx.x & 63;
  int rows = 0, o0 = 0;
  if (lane0 < pk.E) {
    o0 = pk.offsets[lane0];
    rows = pk.offsets[lane0 + 1] - o0;
  }
  if (threadIdx.x < 64) {
    if (lane0 < pk.E) off[lane0] = o0;
    if (lane0 == pk.E - 1) off[pk.E] = o0 + rows;
  }
  int sum = rows, mx = rows;
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    sum += __shfl_xor(sum, d, 64);
    mx = max(mx, __shfl_xor(mx, d, 64));
  }
  block_barrier();   // queues and arguments are in LDS

  RkQueue q;
  q.off = off;
  q.NI = int((pk.n_i + kT - 1) / kT);
  q.NJ = int((pk.n_j + kT - 1) / kT);
  q.per_e = q.NI * q.NJ;
  q.n_tiles = int(pk.n_tiles);
  q.contiguous = __builtin_amdgcn_readfirstlane(int((pk.rk_xcd & 1) && int64_t(mx) * pk.E * 8 <= int64_t(sum) * 9));
  q.chunked = !q.contiguous && (pk.rk_xcd & 2) != 0;
  q.per_xcd = (q.n_tiles + 7) / 8;
  q.xcd = int(blockIdx.x % 8);
  q.nbx = int(gridDim.x / 8);
  q.c0 = q.nbx - 1 - int(blockIdx.x / 8);
  q.jfast = pk.rk_jfast;

  const int nk_m = int(pm.K / KSTEP);   // >= 2 (launcher)
  int cm = 0, ck = 0;                   // positions in the two shares
  auto next_item = [&](ItemMK& it) -> bool {
    TileP tp;
    if (tile_queue_get(tq, cm, tp)) {
      ++cm;
      it = ItemMK{0, tp.e, tp.i0, tp.j0, tp.j_end, 0, nk_m};
      return true;
    }
    TileK tk;
    if (!rk_next_long(q, ck, tk, KSTEP)) return false;
    it = ItemMK{1, tk.e, tk.i0, tk.j0, 0, tk.k_lo, tk.nk};
    return true;
  };
  auto streams = [&](const ItemMK& it) {
    if (it.k_mode) {
      const Operand Q = uniform_operand(&plk->Q), P = uniform_operand(&plk->P);
      return tile_streams<KIND>(Q, P, rfl64(plk->n_i), TileP{0, it.i0, it.j0, int(rfl64(plk->n_j))}, w);
    }
    const Operand Q = uniform_operand(&plm->Q), P = uniform_operand(&plm->P);
    return tile_streams<KIND>(Q, P, rfl64(plm->n_i), TileP{it.e, it.i0, it.j0, it.j_end}, w);
  };
  const uint32_t smem_lds = lds_addr(smem);
  uint8_t* const W = smem + 2 * SM::kStage + w.wave * 2048;

  auto store = [&](void* C, int64_t ldC, int out_f32, int64_t row0, int64_t col0, const v16f (&acc)[4][2]) {
    WaveCoord we = w;
    we.lane = fresh_lane();
    we.lrow = we.lane & 31;
    we.lhalf = we.lane >> 5;
    if (!out_f32) {
      store_bf16_passes(acc, W, static_cast<uint16_t*>(C), ldC, row0, col0, we);
    } else {
      float* dst = static_cast<float*>(C) + row0 * ldC + col0 + we.lrow * ldC + 4 * we.lhalf;
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4)
            st_global(dst + b * 32 * ldC + a * 32 + 8 * r4, make_float4(
                acc[a][b][4 * r4], acc[a][b][4 * r4 + 1], acc[a][b][4 * r4 + 2], acc[a][b][4 * r4 + 3]));
    }
  };
  auto epilogue = [&](const ItemMK& it, const v16f (&acc)[4][2]) {
    const int64_t ib = it.i0 + w.wi * 128, jb = it.j0 + w.wj * 64;
    if (it.k_mode) {   // weight gradient: row j (m), column i; rows past `split` to C2
      if (ib >= rfl64(plk->n_i) || jb >= rfl64(plk->n_j)) return;
      const int64_t split = rfl64(plk->split);
      const bool second = uniform_ge(jb, split);
      const int64_t gs = second ? rfl64(plk->c2_gs) : rfl64(plk->c_gs);
      uint8_t* const Cb = static_cast<uint8_t*>(second ? plk->C2 : plk->C);
      const int f32 = __builtin_amdgcn_readfirstlane(plk->out_f32);
      store(Cb + int64_t(it.e) * gs * (f32 ? 4 : 2), rfl64(plk->ldC), f32, second ? jb - split : jb, ib, acc);
    } else {           // dgrad: row j (token), column i
      const int p_rows = it.j_end - it.j0 < kT ? it.j_end - it.j0 : kT;
      if (ib >= rfl64(plm->n_i) || jb >= it.j0 + p_rows) return;
      store(plm->C, rfl64(plm->ldC), __builtin_amdgcn_readfirstlane(plm->out_f32), jb, ib, acc);
    }
  };

  Frag<KIND> f0, f1;
  ItemMK cur;
  if (next_item(cur)) {
    TileStreams S = streams(cur);
    issue_step<KIND>(S.q, S.p, S.sc, cur.k_base, smem_lds, w.wave);
    issue_step<KIND>(S.q, S.p, S.sc, cur.k_base + KSTEP, smem_lds + SM::kStage, w.wave);
    FM_WAIT_VMCNT(KIND == GK_BF16 ? 8 : 9);
    block_barrier();
    read_half<KIND>(smem, 0, f0, w);
    int cur_off = 0;
    for (;;) {
      ItemMK nxt;
      const bool has_next = next_item(nxt);
      v16f acc[4][2];
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;
      auto step = [&](int64_t k) {
        const int nxt_off = SM::kStage - cur_off;
        __builtin_amdgcn_sched_barrier(0);
        read_half<KIND>(smem + cur_off, 1, f1, w);
        if constexpr (KIND == GK_FP8_POW2) {
          f1.sa[0] = f0.sa[0];
          f1.sb[0] = f0.sb[0];
        }
        mma_half<KIND>(f0, acc);
        interleave_half<KIND>();
        __builtin_amdgcn_sched_barrier(0);
        FM_WAIT_VMCNT(0);
        block_barrier();
        issue_read_half0<KIND>(S.q, S.p, S.sc, k, smem_lds + cur_off, w.wave, smem + nxt_off, f0, w);
        mma_half<KIND>(f1, acc);
        interleave_half<KIND>();
        __builtin_amdgcn_sched_barrier(0);
        cur_off = nxt_off;
      };
      const int nk = cur.nk;   // >= 2
#pragma unroll 1
      for (int t = 0; t < nk - 2; ++t) step(int64_t(cur.k_base) + int64_t(t + 2) * KSTEP);
      const int64_t last = int64_t(cur.k_base) + int64_t(nk - 1) * KSTEP;
      if (has_next) S = streams(nxt);
#pragma unroll 1
      for (int t = 0; t < 2; ++t) step(has_next ? int64_t(nxt.k_base) + int64_t(t) * KSTEP : last);
      epilogue(cur, acc);
      if (!has_next) break;
      cur = nxt;
    }
    FM_WAIT_VMCNT(0);
    block_barrier();   // the stages are free again
  }

  // ragged-K tiles of fewer than two K steps, one at a time
  for (int c = 0;; ++c) {
    TileK t;
    if (!rk_tile_at(q, c, t, KSTEP)) break;
    if (t.nk >= 2) continue;
    const ItemMK it{1, t.e, t.i0, t.j0, 0, t.k_lo, t.nk};
    v16f acc[4][2];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;
    if (t.nk == 1) {
      const TileStreams S = streams(it);
      issue_step<KIND>(S.q, S.p, S.sc, t.k_lo, smem_lds, w.wave);
      FM_WAIT_VMCNT(0);
      block_barrier();
      read_half<KIND>(smem, 0, f0, w);
      read_half<KIND>(smem, 1, f1, w);
      if constexpr (KIND == GK_FP8_POW2) {
        f1.sa[0] = f0.sa[0];
        f1.sb[0] = f0.sb[0];
      }
      mma_half<KIND>(f0, acc);
      mma_half<KIND>(f1, acc);
      block_barrier();   // every wave has read the stage before the next tile's DMA
    }
    epilogue(it, acc);
  }
}

// ============================================================================
// Ring variant of the persistent kernels: paired-row operands
// ============================================================================
// In the paired-row layout (FM_GEMM_PAIRED) rows 2p and 2p + 1 of an operand
// share "pair row" p, and each 128-byte piece of a pair row holds 64 K bytes
// of row 2p followed by the same 64 K bytes of row 2p + 1:
//   byte (r, k) at (r >> 1) * 2 ld + (k >> 6) * 128 + (r & 1) * 64 + (k & 63).
// A 64-deep K slab of a tile is then whole 128-byte lines, so the K loop runs
// over half steps (64 deep) through a ring of four LDS slots of 34 KiB (both
// operands and, with even halves, the step's pow2 scales): the DMA of half
// j + 4 is issued when half j's slot is released, and each half step waits
// only for the next half while the two after it stay in flight -- the
// two-stage loop of gemm256p_kernel drains every load at each step, which
// bounds its operand stream (measured on gfx950 with the same tiles: 12.3
// TB/s with one step in flight, 17 TB/s with a second one; 64-byte row pieces
// stay at 12.5 whatever the depth).  [K][N] weights (QNN) need no pairing: a
// 64-deep slab is 64 K rows of 256 bytes.  Each half step has its own barrier.
// Fragments, scales and the MFMA order are those of gemm256p_kernel, so the
// results are bit-identical.
constexpr int kSlotOp = kT * 64;   // one operand, one 64-deep half step
// pow2: each slot holds both operands and, with an even half, the step's
// scales (one fp32 per row and operand).  MX: the slots hold operands only;
// a step's e8m0 scales (4 bytes per row and operand: both halves' blocks) go
// to a ring of three 2 KiB scale slots after them, step t's in slot t % 3, so
// an odd half still finds its step's scales after the even half's slot has
// been refilled.
template <int KIND>
struct SmemR {
  static constexpr bool kMX = KIND == GK_FP8_MX;
  static constexpr int kS = kT * 4;   // scales of one operand, one step
  static constexpr int kP = kSlotOp;
  static constexpr int kSlot = 2 * kSlotOp + (kMX ? 0 : 2 * kS);
  static constexpr int kQS = kMX ? 0 : 2 * kSlotOp, kPS = kQS + kS;   // in the slot (pow2) / scale slot (MX)
  static constexpr int kScaleBase = 4 * kSlot, kScaleSlot = 2 * kS;
  static constexpr int kBytes = 4 * kSlot + (kMX ? 3 * kScaleSlot : 0);
};

// Row r of a paired slot operand: 64 bytes at r * 64, 16-byte chunk c at
// position c ^ ((r / 4) % 4), so the 16 rows one ds_read_b128 pass touches
// fall on 16 distinct 16-byte bank groups.
__device__ __forceinline__ int pr_off(int row, int chunk) { return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4); }
// The NT fragment of read_frag8 (lane half h: K [16h, +16) and [32 + 16h, +16))
__device__ __forceinline__ v8i read_frag8_pr(const uint8_t* base, int r, int lhalf) {
  const v4i x0 = *reinterpret_cast<const v4i*>(base + pr_off(r, lhalf));
  const v4i x1 = *reinterpret_cast<const v4i*>(base + pr_off(r, lhalf + 2));
  return __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
}

// DMA source of one operand for half steps.  Paired NT operand: wave w moves
// rows [32w, 32w + 32) (pairs [16w, 16w + 16)) as two groups of 8 pair rows x
// 128 bytes; lane n takes pair n / 8, row (n / 4) % 2 of the pair, chunk
// (n % 4) ^ ((n / 16) % 4), which lands at LDS row 16 g + n / 4, position n % 4
// of its group g.  [K][N] operand: wave w moves K rows [8w, 8w + 8) as two
// groups of 4 K rows (make_stream_nn's lanes; both parities).
struct RingStream {
  v4i rsrc;
  uint32_t group_bytes;
  uint32_t lane_off[2];
  uint32_t k_half_bytes;   // byte advance per half step
};
__device__ __forceinline__ RingStream make_stream_pr(const uint8_t* base, int64_t ld, int64_t rows, int lane,
                                                     int wave) {
  RingStream s;
  const int last = int(rows / 32) - 1;
  s.rsrc = make_rsrc(base + int64_t(wave < last ? wave : last) * 32 * ld);
  s.group_bytes = uint32_t(16 * ld);
  s.lane_off[0] = s.lane_off[1] =
      uint32_t((lane >> 3) * 2 * ld + ((lane >> 2) & 1) * 64 + (((lane & 3) ^ ((lane >> 4) & 3)) << 4));
  s.k_half_bytes = 128;
  return s;
}
__device__ __forceinline__ RingStream make_stream_nn_half(const uint8_t* base, int64_t ld, int lane, int wave) {
  RingStream s;
  s.rsrc = make_rsrc(base + int64_t(wave) * 8 * ld);
  s.group_bytes = uint32_t(4 * ld);
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int row = lane >> 4, kk = 4 * par + row;
    s.lane_off[par] = uint32_t(row * ld + 16 * ((lane & 15) ^ (2 * kk)));
  }
  s.k_half_bytes = uint32_t(64 * ld);
  return s;
}

// [K][N] operand in the paired-row layout (K rows 2p, 2p + 1 interleaved in
// 64-byte pieces of N): the same LDS layout as make_stream_nn_half (K row k at
// k * 256, 16-byte chunk c at position c ^ 2 (k % 8)), so lane n of group u
// (K rows 4u .. 4u + 3 of the wave's 8) fetches K row kr = n / 16 of the
// group, logical chunk c = (n % 16) ^ 2 (4u + kr): pair kr / 2, piece kr % 2
// of the 128-byte line of N block c / 4.  A group's 64 lanes cover 8 whole
// lines.  `base` points at N column 0 of the tile in K row 0.
__device__ __forceinline__ RingStream make_stream_nn_half_paired(const uint8_t* base, int64_t ld, int lane,
                                                                 int wave) {
  RingStream s;
  s.rsrc = make_rsrc(base + int64_t(wave) * 8 * ld);
  s.group_bytes = uint32_t(4 * ld);
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int kr = lane >> 4, c = (lane & 15) ^ (2 * (4 * par + kr));
    s.lane_off[par] = uint32_t((kr >> 1) * 2 * ld + (kr & 1) * 64 + (c >> 2) * 128 + (c & 3) * 16);
  }
  s.k_half_bytes = uint32_t(64 * ld);
  return s;
}

struct RingStreams {
  RingStream q, p;
  ScaleSrc sc;
};

template <int KIND, bool QNN, bool QP>
__device__ __forceinline__ RingStreams ring_streams(const Operand& Q, const Operand& P, int64_t n_i, const TileP& t,
                                                   const WaveCoord& w) {
  RingStreams s;
  const int64_t q_rows = n_i - t.i0 < kT ? n_i - t.i0 : kT;
  const int64_t p_rows = t.j_end - t.j0 < kT ? t.j_end - t.j0 : kT;
  const int lane = fresh_lane();
  if constexpr (QNN && QP)   // tile column i0 (a multiple of 256): N block i0 / 64 of every pair row
    s.q = make_stream_nn_half_paired(Q.p + int64_t(t.e) * Q.gs + (int64_t(t.i0) >> 6) * 128, Q.ld, lane, w.wave);
  else if constexpr (QNN) s.q = make_stream_nn_half(Q.p + int64_t(t.e) * Q.gs + int64_t(t.i0), Q.ld, lane, w.wave);
  else s.q = make_stream_pr(Q.p + int64_t(t.e) * Q.gs + t.i0 * Q.ld, Q.ld, q_rows, lane, w.wave);
  s.p = make_stream_pr(P.p + int64_t(t.j0) * P.ld, P.ld, p_rows, lane, w.wave);
  // waves 0-3 stream the weights' scales, 4-7 the tokens': the fields are
  // selected by value (a select of the two operands' addresses would put the
  // kernel arguments in scratch memory)
  const int li = (w.wave & 3) * 64 + lane;
  const bool wq = w.wave < 4;
  Operand so;
  so.s = wq ? Q.s : P.s;
  so.s_row = wq ? Q.s_row : P.s_row;
  so.s_kb = wq ? Q.s_kb : P.s_kb;
  so.s_gs = wq ? Q.s_gs : P.s_gs;
  so.s_shift = wq ? Q.s_shift : P.s_shift;
  s.sc = make_scale_src<KIND>(so, wq ? int64_t(t.i0) : int64_t(t.j0), wq ? q_rows : p_rows, wq ? t.e : 0,
                              wq ? w.q_mx_k : w.p_mx_k, li, wq ? SmemR<KIND>::kQS : SmemR<KIND>::kPS);
  return s;
}

// A descriptor held in vector registers (the compiler may move the tile's
// streams there between tiles), read back as the wave-uniform value it is.
__device__ __forceinline__ v4i uniform_rsrc(v4i r) {
  v4i u;
  u[0] = __builtin_amdgcn_readfirstlane(r[0]);
  u[1] = __builtin_amdgcn_readfirstlane(r[1]);
  u[2] = __builtin_amdgcn_readfirstlane(r[2]);
  u[3] = __builtin_amdgcn_readfirstlane(r[3]);
  return u;
}

// Piece u of half j's DMA: u = 0..3 the operand groups (even: Q group u / 2,
// odd: P group u / 2), u = 4 the step's scale dword (even halves only) into
// `sdst` (the slot for pow2, the step's scale slot for MX).
__device__ __forceinline__ void issue_piece_r(int u, const RingStreams& S, int64_t j, uint32_t dst, uint32_t sdst,
                                              int wave) {
  const int g = u >> 1;
  if (u == 4) {
    bdma4(uniform_rsrc(S.sc.rsrc), S.sc.voff, __builtin_amdgcn_readfirstlane(uint32_t(j >> 1) * S.sc.k),
          sdst + S.sc.dst);
  } else if (u & 1) {
    const uint32_t soff = __builtin_amdgcn_readfirstlane(g * S.p.group_bytes + uint32_t(j) * S.p.k_half_bytes);
    bdma16(uniform_rsrc(S.p.rsrc), S.p.lane_off[g], soff, dst + kSlotOp + (wave * 2 + g) * 1024);
  } else {
    const uint32_t soff = __builtin_amdgcn_readfirstlane(g * S.q.group_bytes + uint32_t(j) * S.q.k_half_bytes);
    bdma16(uniform_rsrc(S.q.rsrc), S.q.lane_off[g], soff, dst + (wave * 2 + g) * 1024);
  }
}

// Reads the fragments of the half in slot `st` into f, with half j's DMA
// pieces placed between the reads.  EVEN: half j is even (its DMA carries the
// step's scale dword); the parity is a template argument so the loop body
// stays one basic block.  Scales of the half read (the other parity): pow2
// with `scales` (an even half) from the slot; MX always, from the scale slot
// `sst`, blocks 2 RODD + (0, 1) of the step.
template <int KIND, bool QNN, bool EVEN>
__device__ __forceinline__ void issue_read_r(const RingStreams& S, int64_t j, uint32_t dst, uint32_t sdst, int wave,
                                             const uint8_t* st, const uint8_t* sst, bool scales, Frag<KIND>& f,
                                             const WaveCoord& w) {
  using SM = SmemR<KIND>;
  if constexpr (KIND == GK_FP8_MX) {
    constexpr int rodd = EVEN ? 1 : 0;   // the half read has the other parity
    const int blk = 2 * rodd + w.lhalf;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      f.sa[t] = read_mx_scale(sst, SM::kQS, w.wi * 128 + t * 32 + w.lrow, blk, w.q_mx_k);
      if (t < 2) f.sb[t] = read_mx_scale(sst, SM::kPS, w.wj * 64 + t * 32 + w.lrow, blk, w.p_mx_k);
    }
  } else if (scales) {
    f.sa[0] = read_pow2_scales(st, SM::kQS, w.wi * 128, w.lrow);
    const uint2 v = *reinterpret_cast<const uint2*>(
        st + SM::kPS + ((w.wj >> 1) * 128 + w.lrow * 4 + 2 * (w.wj & 1)) * 4);
    f.sb[0] = pack_exp4(v.x, v.y, 0u, 0u);
  }
  if constexpr (EVEN) issue_piece_r(4, S, j, dst, sdst, wave);
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if constexpr (QNN) f.a[t] = read_frag8_nn(st, w.wi * 128 + t * 32, 0, w.lane);
    else f.a[t] = read_frag8_pr(st, w.wi * 128 + t * 32 + w.lrow, w.lhalf);
    issue_piece_r(t, S, j, dst, sdst, wave);
    if (t < 2) f.b[t] = read_frag8_pr(st + kSlotOp, w.wj * 64 + t * 32 + w.lrow, w.lhalf);
  }
}

// One tile of the ring walk: a ragged-M tile (k_mode 0: expert e, weight
// rows i0, token rows j0 .. j_end) or a ragged-K tile (k_mode 1: expert e's
// weight-gradient tile i0, j0 over its tokens); kh0 = first 64-deep half step
// (absolute: a token offset / 64 for ragged-K), nh = half steps.
struct ItemR {
  int k_mode, e, i0, j0, j_end, kh0, nh;
};

// The next tile of the share with at least `min_nk` K steps, from position `c`.
__device__ __forceinline__ bool rk_next_min(const RkQueue& q, int& c, TileK& t, int kstep, int min_nk) {
  for (;;) {
    if (!rk_tile_at(q, c, t, kstep)) return false;
    ++c;
    if (t.nk >= min_nk) return true;
  }
}

// Persistent ring walk over paired-row operands (FP8 pow2): HAS_M -- the
// ragged-M tiles of pm (the per-XCD shares of gemm256p_kernel), HAS_K -- then
// the ragged-K tiles of pk (the shares of gemm256pk_kernel; with HAS_M the
// workgroups of an XCD take them in reverse order, as gemm256pmk_kernel).
// QNN / QP: pm's weights stored [K][N] / paired (ragged-K operands are paired
// [rows][tokens]).  Every tile runs the four-slot ring of half steps and the
// last four refills of a tile fetch the next tile's first four halves;
// ragged-K tiles of one K step come last, one at a time.  No
// expert masks, at most 64 experts, ragged-M K >= 384 (the launcher).
template <int KIND, int MXL, bool HAS_M, bool HAS_K, bool QNN, bool QP>
__global__ __launch_bounds__(512) void gemm256r_kernel(GemmParams pm, GemmParams pk) {
  static_assert(!(HAS_K && QNN), "ragged-K tiles share the NT fragment reads");
  static_assert(KIND == GK_FP8_POW2 || (KIND == GK_FP8_MX && !QNN), "pow2, or MX with [N][K] weights");
  using SM = SmemR<KIND>;
  constexpr bool MX = KIND == GK_FP8_MX;
  constexpr int kSpare = 8 * 2048;   // epilogue staging, 2 KiB per wave
  constexpr int kQueue = 1024;       // ragged-M tile queue
  constexpr int kOff = 512;          // ragged-K offsets copy
  constexpr int kArgs = (sizeof(GemmParams) + 15) / 16 * 16;
  constexpr int kBase = SM::kBytes;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kBase + kSpare + kQueue + kOff + 2 * kArgs];
  int* const qlds = reinterpret_cast<int*>(smem + kBase + kSpare);
  int* const off = reinterpret_cast<int*>(smem + kBase + kSpare + kQueue);
  GemmParams* const plm = reinterpret_cast<GemmParams*>(smem + kBase + kSpare + kQueue + kOff);
  GemmParams* const plk = reinterpret_cast<GemmParams*>(smem + kBase + kSpare + kQueue + kOff + kArgs);
  if (threadIdx.x == 0) {
    *plm = pm;
    *plk = pk;
  }

  WaveCoord w;
  w.lane = threadIdx.x & 63;
  w.wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  w.wi = w.wave >> 2;
  w.wj = w.wave & 3;
  w.lrow = w.lane & 31;
  w.lhalf = w.lane >> 5;
  w.q_mx_k = MX && (MXL & 1) != 0;
  w.p_mx_k = MX && (MXL & 2) != 0;

  TileQueue tq;
  if constexpr (HAS_M) tile_queue_init(pm, tq, qlds);
  int sum = 0, mx = 0;
  if constexpr (HAS_K) {
    const int lane0 = threadIdx.x & 63;
    int rows = 0, o0 = 0;
    if (lane0 < pk.E) {
      o0 = pk.offsets[lane0];
      rows = pk.offsets[lane0 + 1] - o0;
    }
    if (threadIdx.x < 64) {
      if (lane0 < pk.E) off[lane0] = o0;
      if (lane0 == pk.E - 1) off[pk.E] = o0 + rows;
    }
    sum = rows;
    mx = rows;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      sum += __shfl_xor(sum, d, 64);
      mx = max(mx, __shfl_xor(mx, d, 64));
    }
  }
  block_barrier();   // queues and arguments are in LDS

  RkQueue q{};
  if constexpr (HAS_K) {
    q.off = off;
    q.NI = int((pk.n_i + kT - 1) / kT);
    q.NJ = int((pk.n_j + kT - 1) / kT);
    q.per_e = q.NI * q.NJ;
    q.n_tiles = int(pk.n_tiles);
    q.contiguous = __builtin_amdgcn_readfirstlane(int((pk.rk_xcd & 1) && int64_t(mx) * pk.E * 8 <= int64_t(sum) * 9));
    q.chunked = !q.contiguous && (pk.rk_xcd & 2) != 0;
    q.per_xcd = (q.n_tiles + 7) / 8;
    q.xcd = int(blockIdx.x % 8);
    q.nbx = int(gridDim.x / 8);
    q.c0 = HAS_M ? q.nbx - 1 - int(blockIdx.x / 8) : int(blockIdx.x / 8);
    q.jfast = pk.rk_jfast;
  }

  const int nh_m = HAS_M ? int(pm.K / 64) : 0;   // >= 6 (launcher)
  int cm = 0, ck = 0;                              // positions in the two shares
  auto next_item = [&](ItemR& it) -> bool {
    if constexpr (HAS_M) {
      TileP tp;
      if (tile_queue_get(tq, cm, tp)) {
        ++cm;
        it = ItemR{0, tp.e, tp.i0, tp.j0, tp.j_end, 0, nh_m};
        return true;
      }
    }
    if constexpr (HAS_K) {
      TileK tk;
      if (rk_next_min(q, ck, tk, 128, 2)) {
        it = ItemR{1, tk.e, tk.i0, tk.j0, 0, tk.k_lo / 64, 2 * tk.nk};
        return true;
      }
    }
    return false;
  };
  auto streams = [&](const ItemR& it) -> RingStreams {
    if (HAS_K && (!HAS_M || it.k_mode)) {
      const Operand Q = uniform_operand(&plk->Q), P = uniform_operand(&plk->P);
      return ring_streams<KIND, false, true>(Q, P, rfl64(plk->n_i), TileP{0, it.i0, it.j0, int(rfl64(plk->n_j))}, w);
    }
    const Operand Q = uniform_operand(&plm->Q), P = uniform_operand(&plm->P);
    return ring_streams<KIND, QNN, QP>(Q, P, rfl64(plm->n_i), TileP{it.e, it.i0, it.j0, it.j_end}, w);
  };
  const uint32_t smem_lds = lds_addr(smem);
  uint8_t* const W = smem + kBase + w.wave * 2048;

  // returns a lower bound of the output store instructions the wave issued:
  // 16 x 16 bytes of bf16 (the unaligned path's 8-byte pairs may be merged
  // into 16-byte stores), 32 x 16 bytes of fp32; a count above the issued
  // stores would let the next tile read a slot before its data landed
  auto store = [&](void* C, int64_t ldC, int out_f32, int64_t row0, int64_t col0, const v16f (&acc)[4][2]) -> int {
    WaveCoord we = w;
    we.lane = fresh_lane();
    we.lrow = we.lane & 31;
    we.lhalf = we.lane >> 5;
    if (!out_f32) {
      store_bf16_passes(acc, W, static_cast<uint16_t*>(C), ldC, row0, col0, we);
      return 16;
    } else {
      float* dst = static_cast<float*>(C) + row0 * ldC + col0 + we.lrow * ldC + 4 * we.lhalf;
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4)
            st_global(dst + b * 32 * ldC + a * 32 + 8 * r4, make_float4(
                acc[a][b][4 * r4], acc[a][b][4 * r4 + 1], acc[a][b][4 * r4 + 2], acc[a][b][4 * r4 + 3]));
      return 32;
    }
  };
  // returns the wave's output store instructions (wave-uniform)
  auto epilogue = [&](const ItemR& it, const v16f (&acc)[4][2]) -> int {
    const int64_t ib = it.i0 + w.wi * 128, jb = it.j0 + w.wj * 64;
    if (HAS_K && (!HAS_M || it.k_mode)) {   // weight gradient: row j (m), column i; rows past `split` to C2
      if (ib >= rfl64(plk->n_i) || jb >= rfl64(plk->n_j)) return 0;
      const int64_t split = rfl64(plk->split);
      const bool second = uniform_ge(jb, split);
      const int64_t gs = second ? rfl64(plk->c2_gs) : rfl64(plk->c_gs);
      uint8_t* const Cb = static_cast<uint8_t*>(second ? plk->C2 : plk->C);
      const int f32 = __builtin_amdgcn_readfirstlane(plk->out_f32);
      return store(Cb + int64_t(it.e) * gs * (f32 ? 4 : 2), rfl64(plk->ldC), f32, second ? jb - split : jb, ib,
                   acc);
    } else {   // dgrad / forward: row j (token), column i
      const int p_rows = it.j_end - it.j0 < kT ? it.j_end - it.j0 : kT;
      if (ib >= rfl64(plm->n_i) || jb >= it.j0 + p_rows) return 0;
      return store(plm->C, rfl64(plm->ldC), __builtin_amdgcn_readfirstlane(plm->out_f32), jb, ib, acc);
    }
  };
  auto zero = [](v16f (&acc)[4][2]) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;
  };
  auto slot = [&](int g) { return smem + (g & 3) * SM::kSlot; };
  auto slot_lds = [&](int g) { return smem_lds + uint32_t(g & 3) * SM::kSlot; };
  // MX: step t's scales in scale slot t % 3 (pow2: in the even half's slot)
  auto sslot = [&](int t3) { return smem + SM::kScaleBase + t3 * SM::kScaleSlot; };
  auto sslot_lds = [&](int t3) { return smem_lds + uint32_t(SM::kScaleBase + t3 * SM::kScaleSlot); };
  // the scale target of half g's DMA (its step's scale slot t3 for MX)
  auto sdst = [&](int g, int t3) { return MX ? sslot_lds(t3) : slot_lds(g); };
  // the fragments and scales of an even half (the step's first) in slot g
  auto read_even = [&](int g, int t3, Frag<KIND>& f) {
    const uint8_t* st = slot(g);
    if constexpr (MX) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f.sa[t] = read_mx_scale(sslot(t3), SM::kQS, w.wi * 128 + t * 32 + w.lrow, w.lhalf, w.q_mx_k);
        if (t < 2) f.sb[t] = read_mx_scale(sslot(t3), SM::kPS, w.wj * 64 + t * 32 + w.lrow, w.lhalf, w.p_mx_k);
      }
    } else {
      f.sa[0] = read_pow2_scales(st, SM::kQS, w.wi * 128, w.lrow);
      const uint2 v = *reinterpret_cast<const uint2*>(
          st + SM::kPS + ((w.wj >> 1) * 128 + w.lrow * 4 + 2 * (w.wj & 1)) * 4);
      f.sb[0] = pack_exp4(v.x, v.y, 0u, 0u);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if constexpr (QNN) f.a[t] = read_frag8_nn(st, w.wi * 128 + t * 32, 0, w.lane);
      else f.a[t] = read_frag8_pr(st, w.wi * 128 + t * 32 + w.lrow, w.lhalf);
      if (t < 2) f.b[t] = read_frag8_pr(st + kSlotOp, w.wj * 64 + t * 32 + w.lrow, w.lhalf);
    }
  };
  // the odd half (its step's second) in slot g, scales from scale slot t3 (MX)
  auto read_odd = [&](int g, int t3, Frag<KIND>& f) {
    const uint8_t* st = slot(g);
    if constexpr (MX) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f.sa[t] = read_mx_scale(sslot(t3), SM::kQS, w.wi * 128 + t * 32 + w.lrow, 2 + w.lhalf, w.q_mx_k);
        if (t < 2) f.sb[t] = read_mx_scale(sslot(t3), SM::kPS, w.wj * 64 + t * 32 + w.lrow, 2 + w.lhalf, w.p_mx_k);
      }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      f.a[t] = read_frag8_pr(st, w.wi * 128 + t * 32 + w.lrow, w.lhalf);
      if (t < 2) f.b[t] = read_frag8_pr(st + kSlotOp, w.wj * 64 + t * 32 + w.lrow, w.lhalf);
    }
  };

  Frag<KIND> f0, f1;   // f0: even halves (with the step's scales), f1: odd halves
  ItemR cur;
  if (next_item(cur)) {
    RingStreams S = streams(cur);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int v = 0; v < 5; ++v)
        if (v < 4 || (u & 1) == 0) issue_piece_r(v, S, cur.kh0 + u, slot_lds(u), sdst(u, u >> 1), w.wave);
    }
    FM_WAIT_VMCNT(13);   // half 0 landed (halves 1-3: 4 + 5 + 4 pieces in flight)
    block_barrier();
    read_even(0, 0, f0);
    int gs = 0;     // ring slot of the current even half (0 or 2)
    int ss = 0;     // MX: scale slot of the current step (0, 1, 2)
    int pend = 0;   // output stores of the last epilogue (issued after this tile's halves 1-3)
    for (;;) {
      ItemR nxt;
      const bool has_next = next_item(nxt);
      v16f acc[4][2];
      zero(acc);
      // Two half steps: the even half's MFMAs (f0) while the odd half is read
      // into f1 and absolute half jn (even; with the scales of two steps on)
      // is issued into the even slot, then the odd half's MFMAs while the next
      // even half is read into f0 and jn + 1 is issued into the odd slot.
      // `first`: the tile's first pair, after an epilogue whose `pend` output
      // stores count in vmcnt too: vector memory operations complete in issue
      // order, so the odd half has landed once at most the two halves after
      // it and those stores remain.
      auto pair = [&](int64_t jn, bool first) {
        const int s2 = ss == 0 ? 2 : ss - 1, s1 = ss == 2 ? 0 : ss + 1;   // (ss + 2) % 3, (ss + 1) % 3
        __builtin_amdgcn_sched_barrier(0);
        const int after = first ? pend : 0;   // wave-uniform
        if (after >= 32) FM_WAIT_VMCNT(9 + 32);
        else if (after >= 16) FM_WAIT_VMCNT(9 + 16);
        else FM_WAIT_VMCNT(9);   // the odd half landed (the two halves after it in flight)
        block_barrier();         // every wave has read the even half: its slot is free
        issue_read_r<KIND, QNN, true>(S, jn, slot_lds(gs), sdst(gs, s2), w.wave, slot(gs + 1), sslot(ss), false,
                                      f1, w);
        if constexpr (!MX) {
          f1.sa[0] = f0.sa[0];
          f1.sb[0] = f0.sb[0];
        }
        mma_half<KIND>(f0, acc);
        interleave_half<KIND, QNN>();
        __builtin_amdgcn_sched_barrier(0);
        FM_WAIT_VMCNT(9);
        block_barrier();
        issue_read_r<KIND, QNN, false>(S, jn + 1, slot_lds(gs + 1), 0, w.wave, slot(gs + 2), sslot(s1), true,
                                       f0, w);
        mma_half<KIND>(f1, acc);
        interleave_half<KIND, QNN>();
        __builtin_amdgcn_sched_barrier(0);
        gs = (gs + 2) & 3;
        ss = s1;
      };
      const int nh = cur.nh;   // >= 4
      const int64_t kh0 = cur.kh0;
#pragma unroll 1
      for (int j = 0; j < nh - 4; j += 2) pair(kh0 + j + 4, j == 0);
      if (has_next) S = streams(nxt);
      // the last four halves: the next tile's halves 0-3 (the last tile
      // re-issues its own last two halves, whose slots nothing reads again);
      // a tile of four halves has only these
      const int64_t kn0 = has_next ? int64_t(nxt.kh0) : kh0 + nh - 2;
#pragma unroll 1
      for (int j = 0; j < 4; j += 2) pair(has_next ? kn0 + j : kn0, nh == 4 && j == 0);   // a loop: one block per pair
      pend = __builtin_amdgcn_readfirstlane(epilogue(cur, acc));
      if (!has_next) break;
      cur = nxt;
    }
    FM_WAIT_VMCNT(0);
    block_barrier();   // the slots are free again
  }

  if constexpr (HAS_K) {
    // ragged-K tiles of one K step (or none), one at a time
    for (int c = 0;; ++c) {
      TileK t;
      if (!rk_tile_at(q, c, t, 128)) break;
      if (t.nk >= 2) continue;
      const ItemR it{1, t.e, t.i0, t.j0, 0, t.k_lo / 64, 2 * t.nk};
      v16f acc[4][2];
      zero(acc);
      if (t.nk > 0) {
        const RingStreams S = streams(it);
        for (int u = 0; u < it.nh; ++u)
#pragma unroll
          for (int v = 0; v < 5; ++v)
            if (v < 4 || (u & 1) == 0) issue_piece_r(v, S, it.kh0 + u, slot_lds(u), sdst(u, u >> 1), w.wave);
        FM_WAIT_VMCNT(0);
        block_barrier();
        for (int u = 0; u < it.nh; u += 2) {
          read_even(u, u >> 1, f0);
          read_odd(u + 1, u >> 1, f1);
          if constexpr (!MX) {
            f1.sa[0] = f0.sa[0];
            f1.sb[0] = f0.sb[0];
          }
          mma_half<KIND>(f0, acc);
          mma_half<KIND>(f1, acc);
        }
        block_barrier();   // every wave has read the slots before the next tile's DMA
      }
      epilogue(it, acc);
    }
  }
}

// ============================================================================
// 256 x 128 kernel: FP8_F32 (fp32 block scales, promotion per 128-deep block)
// ============================================================================
constexpr int kBI = 256;   // workgroup tile along i (weight rows / M)
constexpr int kBJ = 128;   // workgroup tile along j (tokens / N)

struct SmemF32 {
  static constexpr int kQ = kBI * 128;                 // operand bytes per stage
  static constexpr int kP = kBJ * 128;
  static constexpr int kQS = kBI * 4;                  // scale bytes per stage
  static constexpr int kPS = kBI * 4;                  // 256 slots, the upper 128 unused
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

__device__ __forceinline__ void f32_issue(const TileSrc& src, int64_t k, uint8_t* stage, int wave) {
  using SM = SmemF32;
#pragma unroll
  for (int u = 0; u < 8; ++u) dma16(src.q[u] + k, stage + (wave * 8 + u) * 1024);
#pragma unroll
  for (int u = 0; u < 4; ++u) dma16(src.p[u] + k, stage + SM::kQ + (wave * 4 + u) * 1024);
  const int64_t ks = k / 128;
  dma4(src.qs + ks * src.qs_k, stage + SM::kQ + SM::kP + wave * 256);
  dma4(src.ps + ks * src.ps_k, stage + SM::kQ + SM::kP + SM::kQS + wave * 256);
}

// One 128-deep K step from a stage: 4 x 2 MFMA 32x32 blocks per wave, each
// 128-deep partial sum promoted with the product of the block scales.
template <int MODE>
__device__ __forceinline__ void f32_compute(const uint8_t* st, v16f (&acc)[4][2], int wi, int wj,
                                            int lrow, int lhalf) {
  using SM = SmemF32;
  const uint8_t* lq = st;
  const uint8_t* lp = st + SM::kQ;
  const float* qs = reinterpret_cast<const float*>(st + SM::kQ + SM::kP);
  const float* ps = reinterpret_cast<const float*>(st + SM::kQ + SM::kP + SM::kQS);
  v8i fa[2][4], fb[2][2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int t = 0; t < 4; ++t) fa[ks][t] = read_frag8(lq, wi * 128 + t * 32 + lrow, ks, lhalf);
#pragma unroll
    for (int t = 0; t < 2; ++t) fb[ks][t] = read_frag8(lp, wj * 64 + t * 32 + lrow, ks, lhalf);
  }
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
        const float s = qs[wi * 128] * sp;  // a wave's 128 rows are one 128x128 weight block
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][b][r] += part[r] * s;
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int ii = wi * 128 + a * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
          acc[a][b][r] += part[r] * (qs[ii] * sp);
        }
      }
    }
}

template <int MODE>
__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmParams p) {
  using SM = SmemF32;
  constexpr int NLOAD = 14;   // DMA instructions per wave per step
  // three pipeline stages of one K step each (operands + scales)
  __shared__ __attribute__((aligned(1024))) uint8_t smem[3 * SM::kStage];
  uint8_t* const smem0 = smem;
  uint8_t* const smem1 = smem + SM::kStage;
  uint8_t* const smem2 = smem + 2 * SM::kStage;

  // ---------------------------------------------------------- tile decode ----
  // ragged-M: the valid 128-row tiles [0, offsets[E] / 128) split into one
  // contiguous range per XCD; ragged-K: tiles in launch order (as above).
  int64_t e = -1, i0 = 0, j0 = 0, k_lo, k_hi;
  const int64_t NI = (p.n_i + kBI - 1) / kBI;
  int64_t L;
  // 128-row tiles of unmasked experts only (see the 256-tile kernel)
  auto unmasked = [&](int x) { return p.mask == nullptr || p.mask[x] == p.mask_want; };
  int64_t MT = 0;
  if (MODE == GM_RAGGED_M) {
    for (int x = 0; x < p.E; ++x)
      if (unmasked(x)) MT += (p.offsets[x + 1] - p.offsets[x]) / kBJ;
    const int64_t n_valid = MT * NI;
    const int64_t per_xcd = (n_valid + 7) / 8;
    const int64_t k = blockIdx.x / 8;
    if (k >= per_xcd) return;
    L = int64_t(blockIdx.x % 8) * per_xcd + k;
    if (L >= n_valid) return;
  } else {
    L = blockIdx.x;
    if (L >= p.n_tiles) return;
  }
  if (MODE == GM_RAGGED_M) {
    const int64_t group = L / (kGroupM * NI);
    const int64_t first = group * kGroupM;
    const int64_t gsz = MT - first < kGroupM ? MT - first : kGroupM;
    int64_t mt = first + (L % gsz);
    const int64_t nt = (L % (kGroupM * NI)) / gsz;
    for (int x = 0; x < p.E; ++x) {
      const int64_t o0 = p.offsets[x];
      const int64_t cnt = unmasked(x) ? (p.offsets[x + 1] - o0) / kBJ : 0;
      if (mt < cnt) {
        e = x;
        j0 = o0 + mt * kBJ;
        break;
      }
      mt -= cnt;
    }
    if (e < 0) return;
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
    src.q[u] = p.Q.p + (q_group * p.Q.gs + gr * p.Q.ld) + ch * 16;
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int c = (wave * 4 + u) * 64 + lane;
    const int row = c >> 3, ch = (c & 7) ^ lds_swz(row);
    src.p[u] = p.P.p + ((j0 + row) * p.P.ld) + ch * 16;
  }
  // Scales: one row per lane, Q 256 rows, P 128 rows (lanes for P rows 128-255
  // re-read row 127 into unused slots, so every wave issues the same loads).
  {
    const int qi = wave * 64 + lane;
    int64_t gr = i0 + qi;
    gr = gr < i_last ? gr : i_last;
    src.qs = static_cast<const uint8_t*>(p.Q.s) + (q_group * p.Q.s_gs + (gr >> p.Q.s_shift) * p.Q.s_row) * 4;
    const int pc = qi < kBJ ? qi : kBJ - 1;
    src.ps = static_cast<const uint8_t*>(p.P.s) + ((j0 + pc) >> p.P.s_shift) * p.P.s_row * 4;
    src.qs_k = p.Q.s_kb * 4;
    src.ps_k = p.P.s_kb * 4;
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
  // passed the barrier that follows its last read of it.
  const int64_t nk = (k_hi - k_lo) / 128;
  if (nk > 0) f32_issue(src, k_lo, smem0, wave);
  if (nk > 1) f32_issue(src, k_lo + 128, smem1, wave);
  // Main loop: steps with a successor, whose loads are always in flight here,
  // so an unconditional vmcnt(NLOAD) retires exactly the current stage's DMA.
  int64_t t = 0;
  while (t + 1 < nk) {
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      if (t + 1 >= nk) break;
      FM_WAIT_VMCNT(NLOAD);
      block_barrier();
      uint8_t* nxt = u == 0 ? smem2 : (u == 1 ? smem0 : smem1);
      const uint8_t* cur = u == 0 ? smem0 : (u == 1 ? smem1 : smem2);
      // unconditional: at t = nk-2 this re-reads step nk-1 into the stage of
      // step nk, which is never read
      const int64_t tn = t + 2 < nk ? t + 2 : nk - 1;
      f32_issue(src, k_lo + tn * 128, nxt, wave);
      f32_compute<MODE>(cur, acc, wi, wj, lrow, lhalf);
      ++t;
    }
  }
  if (t < nk) {  // last step: nothing else in flight
    FM_WAIT_VMCNT(0);
    block_barrier();
    const int sidx = int(t % 3);
    const uint8_t* cur = sidx == 0 ? smem0 : (sidx == 1 ? smem1 : smem2);
    f32_compute<MODE>(cur, acc, wi, wj, lrow, lhalf);
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
            st_global(dst,
                make_float4(acc[a][b][4 * q], acc[a][b][4 * q + 1], acc[a][b][4 * q + 2], acc[a][b][4 * q + 3]));
          } else {
            uint16_t* dst = static_cast<uint16_t*>(p.C) + j * p.ldC + i;
            uint2 v;
            v.x = hw_bf16x2(acc[a][b][4 * q], acc[a][b][4 * q + 1]);
            v.y = hw_bf16x2(acc[a][b][4 * q + 2], acc[a][b][4 * q + 3]);
            st_global(dst, v);
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
          if (p.out_f32) st_global(static_cast<float*>(base) + off, acc[a][b][r]);
          else st_global(static_cast<uint16_t*>(base) + off, f32_to_bf16(acc[a][b][r]));
        }
      }
    }
}

// ============================================================================
// launch
// ============================================================================
// FM_RK_XCD=0: ragged-K launches keep their tiles in launch order even for
// balanced experts (read once).
inline bool gemm_rk_xcd_split() {
  static const bool on = [] {
    const char* e = getenv("FM_RK_XCD");
    return e == nullptr || atoi(e) != 0;
  }();
  return on;
}

// Persistent ragged-K launches over unbalanced experts hand each XCD chunks of
// consecutive tiles (see rk_tile_at) unless FM_RK_CHUNKED=0 (read once).
inline bool gemm_rk_chunked() {
  static const bool on = [] {
    const char* e = getenv("FM_RK_CHUNKED");
    return e == nullptr ? kRkChunkedDefault : atoi(e) != 0;
  }();
  return on;
}

// fm_grouped_gemm_ragged_m_k runs its two launches as one grid unless
// FM_GEMM_MK=0 (then back to back; read once).
inline bool gemm_mk_one_grid() {
  static const bool on = [] {
    const char* e = getenv("FM_GEMM_MK");
    return e == nullptr || atoi(e) != 0;
  }();
  return on;
}

// Unmasked, unsplit BF16, FP8 pow2 and MX ragged-K launches with at most 64
// experts are persistent unless FM_GEMM_PERSISTENT_K=0 (read once).
inline bool gemm_persistent_k() {
  static const bool on = [] {
    const char* e = getenv("FM_GEMM_PERSISTENT_K");
    return e == nullptr || atoi(e) != 0;
  }();
  return on;
}

// Ragged-M launches are persistent unless FM_GEMM_PERSISTENT=0 (read once).
inline bool gemm_persistent() {
  static const bool on = [] {
    const char* e = getenv("FM_GEMM_PERSISTENT");
    return e == nullptr || atoi(e) != 0;
  }();
  return on;
}

// Ragged-M tile order within a group of token tiles.  Weight tiles fastest
// when one expert's weight operand fits an eighth of the 256 MiB Infinity
// Cache (each XCD walks about one expert at a time, so eight of them must
// stay cached for the later rounds to find their weight tiles there); token
// tiles fastest otherwise, so each weight tile is fetched once per group.
// FM_GEMM_ORDER=t / =w forces either order (read once).
constexpr int64_t kWeightFastMaxBytes = int64_t(32) << 20;
inline bool gemm_weight_fast(int64_t weight_bytes) {
  static const int forced = [] {
    const char* e = getenv("FM_GEMM_ORDER");
    return e == nullptr ? 0 : e[0] == 't' ? 1 : e[0] == 'w' ? 2 : 0;
  }();
  return forced == 0 ? weight_bytes <= kWeightFastMaxBytes : forced == 2;
}

// Persistent ragged-M launch: one workgroup per CU (a multiple of 8, one
// share per XCD), at most one per 256 x 256 tile of the host bound.
inline void launch256p(int kind, const GemmParams& p, hipStream_t s) {
  const int64_t slots = int64_t(device_cus() / 8 > 0 ? device_cus() / 8 : 1) * 8;
  const int64_t want = (p.n_tiles + 7) / 8 * 8;
  const dim3 grid(unsigned(want < slots ? want : slots)), block(512);
  switch (kind) {
    case GK_BF16:
      if (p.q_nn) hipLaunchKernelGGL((gemm256p_kernel<GK_BF16, 0, true>), grid, block, 0, s, p);
      else hipLaunchKernelGGL((gemm256p_kernel<GK_BF16>), grid, block, 0, s, p);
      break;
    case GK_FP8_POW2:
      if (p.paired) {
        if (p.q_nn && p.paired == 2)
          hipLaunchKernelGGL((gemm256r_kernel<GK_FP8_POW2, 0, true, false, true, true>), grid, block, 0, s, p, p);
        else if (p.q_nn)
          hipLaunchKernelGGL((gemm256r_kernel<GK_FP8_POW2, 0, true, false, true, false>), grid, block, 0, s, p, p);
        else hipLaunchKernelGGL((gemm256r_kernel<GK_FP8_POW2, 0, true, false, false, true>), grid, block, 0, s, p, p);
      } else if (p.q_nn) {
        hipLaunchKernelGGL((gemm256p_kernel<GK_FP8_POW2, 0, true>), grid, block, 0, s, p);
      } else {
        hipLaunchKernelGGL((gemm256p_kernel<GK_FP8_POW2>), grid, block, 0, s, p);
      }
      break;
    default: {
      const int mxl = (p.Q.s_kb != 1 ? 1 : 0) | (p.P.s_kb != 1 ? 2 : 0);
      if (p.paired) {   // [N][K] weights and tokens paired
        switch (mxl) {
          case 0: hipLaunchKernelGGL((gemm256r_kernel<GK_FP8_MX, 0, true, false, false, true>), grid, block, 0, s, p, p); break;
          case 1: hipLaunchKernelGGL((gemm256r_kernel<GK_FP8_MX, 1, true, false, false, true>), grid, block, 0, s, p, p); break;
          case 2: hipLaunchKernelGGL((gemm256r_kernel<GK_FP8_MX, 2, true, false, false, true>), grid, block, 0, s, p, p); break;
          default: hipLaunchKernelGGL((gemm256r_kernel<GK_FP8_MX, 3, true, false, false, true>), grid, block, 0, s, p, p); break;
        }
        break;
      }
      switch (mxl) {
        case 0: hipLaunchKernelGGL((gemm256p_kernel<GK_FP8_MX, 0>), grid, block, 0, s, p); break;
        case 1: hipLaunchKernelGGL((gemm256p_kernel<GK_FP8_MX, 1>), grid, block, 0, s, p); break;
        case 2: hipLaunchKernelGGL((gemm256p_kernel<GK_FP8_MX, 2>), grid, block, 0, s, p); break;
        default: hipLaunchKernelGGL((gemm256p_kernel<GK_FP8_MX, 3>), grid, block, 0, s, p); break;
      }
    }
  }
}

// Persistent ragged-K launch: one workgroup per CU (a multiple of 8), at most
// one per tile.
inline void launch256pk(int kind, const GemmParams& p, hipStream_t s) {
  const int64_t slots = int64_t(device_cus() / 8 > 0 ? device_cus() / 8 : 1) * 8;
  const int64_t want = (p.n_tiles + 7) / 8 * 8;
  const dim3 grid(unsigned(want < slots ? want : slots)), block(512);
  if (kind == GK_BF16) {
    hipLaunchKernelGGL((gemm256pk_kernel<GK_BF16>), grid, block, 0, s, p);
  } else if (kind == GK_FP8_POW2) {
    hipLaunchKernelGGL((gemm256pk_kernel<GK_FP8_POW2>), grid, block, 0, s, p);
  } else {
    const int mxl = (p.Q.s_kb != 1 ? 1 : 0) | (p.P.s_kb != 1 ? 2 : 0);
    switch (mxl) {
      case 0: hipLaunchKernelGGL((gemm256pk_kernel<GK_FP8_MX, 0>), grid, block, 0, s, p); break;
      case 1: hipLaunchKernelGGL((gemm256pk_kernel<GK_FP8_MX, 1>), grid, block, 0, s, p); break;
      case 2: hipLaunchKernelGGL((gemm256pk_kernel<GK_FP8_MX, 2>), grid, block, 0, s, p); break;
      default: hipLaunchKernelGGL((gemm256pk_kernel<GK_FP8_MX, 3>), grid, block, 0, s, p); break;
    }
  }
}

template <int MODE>
inline void launch256(int kind, dim3 grid, const GemmParams& p, hipStream_t s) {
  const dim3 block(512);
  switch (kind) {
    case GK_BF16: hipLaunchKernelGGL((gemm256_kernel<GK_BF16, MODE>), grid, block, 0, s, p); break;
    case GK_FP8_POW2: hipLaunchKernelGGL((gemm256_kernel<GK_FP8_POW2, MODE>), grid, block, 0, s, p); break;
    default: {
      const int mxl = (p.Q.s_kb != 1 ? 1 : 0) | (p.P.s_kb != 1 ? 2 : 0);
      switch (mxl) {
        case 0: hipLaunchKernelGGL((gemm256_kernel<GK_FP8_MX, MODE, 0>), grid, block, 0, s, p); break;
        case 1: hipLaunchKernelGGL((gemm256_kernel<GK_FP8_MX, MODE, 1>), grid, block, 0, s, p); break;
        case 2: hipLaunchKernelGGL((gemm256_kernel<GK_FP8_MX, MODE, 2>), grid, block, 0, s, p); break;
        default: hipLaunchKernelGGL((gemm256_kernel<GK_FP8_MX, MODE, 3>), grid, block, 0, s, p); break;
      }
    }
  }
}

// Launch-independent preparation: operand sides, tile count, tile order.
template <int MODE>
int prepare_gemm(int kind, GemmParams& p) {
  if (kind < GK_BF16 || kind > GK_FP8_MX) {
    set_error("grouped gemm: unknown kind %d", kind);
    return 1;
  }
  if (MODE == GM_RAGGED_K && kind != GK_FP8_F32) {
    // the 256 x 256 kernel writes rows along j: put the output's row operand
    // (a_t, M rows) on the P side and its column operand (b_t) on the Q side
    const Operand t = p.P;
    p.P = p.Q;
    p.Q = t;
    const int64_t n = p.n_i;
    p.n_i = p.n_j;
    p.n_j = n;
  }
  const int64_t NI256 = (p.n_i + kT - 1) / kT;
  if (kind == GK_FP8_F32) {
    const int64_t NI = (p.n_i + kBI - 1) / kBI;
    p.n_tiles = MODE == GM_RAGGED_M ? p.m_tiles * NI : int64_t(p.E) * NI * (p.n_j / kBJ);
  } else {
    if (p.splits < 1) p.splits = 1;
    p.n_tiles = MODE == GM_RAGGED_M ? p.j_tiles * NI256
                                    : int64_t(p.E) * NI256 * ((p.n_j + kT - 1) / kT) * p.splits;
  }
  p.rk_xcd = MODE == GM_RAGGED_K ? (gemm_rk_xcd_split() ? 1 : 0) | (gemm_rk_chunked() ? 2 : 0) : 0;
  p.w_fast = MODE == GM_RAGGED_M && gemm_weight_fast(p.n_i * p.K * (kind == GK_BF16 ? 2 : 1)) ? 1 : 0;
  return 0;
}

template <int MODE>
int dispatch_gemm(int kind, GemmParams p, hipStream_t s) {
  if (int rc = prepare_gemm<MODE>(kind, p)) return rc;
  if (p.n_tiles == 0) return 0;
  const dim3 grid(unsigned((p.n_tiles + 7) / 8 * 8)), block(256);
  if (kind == GK_FP8_F32) {
    hipLaunchKernelGGL((gemm_f32_kernel<MODE>), grid, block, 0, s, p);
  } else if (MODE == GM_RAGGED_M && p.E <= 64 && p.K / (kind == GK_BF16 ? 64 : 128) >= 2 &&
             (gemm_persistent() || p.q_nn || p.paired || p.Q.split != INT64_MAX)) {
    launch256p(kind, p, s);
  } else if (MODE == GM_RAGGED_K && p.paired) {
    // paired-row operands (checked by the entry point): the ring walk
    const int64_t slots = int64_t(device_cus() / 8 > 0 ? device_cus() / 8 : 1) * 8;
    const int64_t want = (p.n_tiles + 7) / 8 * 8;
    const dim3 pgrid(unsigned(want < slots ? want : slots)), pblock(512);
    if (kind == GK_FP8_POW2) {
      hipLaunchKernelGGL((gemm256r_kernel<GK_FP8_POW2, 0, false, true, false, true>), pgrid, pblock, 0, s, p, p);
    } else {
      switch ((p.Q.s_kb != 1 ? 1 : 0) | (p.P.s_kb != 1 ? 2 : 0)) {
        case 0: hipLaunchKernelGGL((gemm256r_kernel<GK_FP8_MX, 0, false, true, false, true>), pgrid, pblock, 0, s, p, p); break;
        case 1: hipLaunchKernelGGL((gemm256r_kernel<GK_FP8_MX, 1, false, true, false, true>), pgrid, pblock, 0, s, p, p); break;
        case 2: hipLaunchKernelGGL((gemm256r_kernel<GK_FP8_MX, 2, false, true, false, true>), pgrid, pblock, 0, s, p, p); break;
        default: hipLaunchKernelGGL((gemm256r_kernel<GK_FP8_MX, 3, false, true, false, true>), pgrid, pblock, 0, s, p, p); break;
      }
    }
  } else if (MODE == GM_RAGGED_K && p.splits == 1 && p.mask == nullptr && p.E <= 64 &&
             p.n_tiles < (int64_t(1) << 28) && gemm_persistent_k()) {
    // (its tile walk counts in 32-bit integers)
    launch256pk(kind, p, s);
  } else {
    launch256<MODE>(kind, grid, p, s);
  }
  return check_launch("grouped gemm");
}

inline Operand make_operand(const FmGemmOperand& o) {
  return Operand{static_cast<const uint8_t*>(o.data), o.ld, o.group_stride, o.scale,
                 o.scale_row_stride, o.scale_kb_stride, o.scale_group_stride, o.scale_row_shift,
                 static_cast<const uint8_t*>(o.data2 ? o.data2 : o.data), o.data2 ? o.split_rows : INT64_MAX};
}

inline int check_operand(const FmGemmOperand& o, int kind, const char* name) {
  FM_REQUIRE(o.data != nullptr, "grouped gemm: operand %s is null", name);
  FM_REQUIRE(o.ld % 16 == 0, "grouped gemm: operand %s pitch must be a multiple of 16 elements", name);
  FM_REQUIRE(kind == GK_BF16 || o.scale != nullptr, "grouped gemm: operand %s scales are null", name);
  FM_REQUIRE(o.scale_row_shift >= 0 && o.scale_row_shift <= 7, "grouped gemm: operand %s scale_row_shift out of range", name);
  // the DMA addresses a wave's 64-row slab with 32-bit offsets from its base
  FM_REQUIRE(o.ld * (kind == GK_BF16 ? 2 : 1) <= (int64_t(1) << 25),
             "grouped gemm: operand %s pitch exceeds 32 MiB per row", name);
  return 0;
}

// Largest scale byte offset a lane can address from its group base (rows of
// the operand, contraction length), kept below 2^32 for the 32-bit buffer
// offsets of the DMA.
inline int check_scale_span(const FmGemmOperand& o, int kind, int64_t rows, int64_t K, const char* name) {
  if (kind == GK_BF16) return 0;
  const int64_t sb = kind == GK_FP8_MX ? 1 : 4;
  const int64_t blk = kind == GK_FP8_MX ? 32 : 128;
  const int64_t span = ((rows >> o.scale_row_shift) + 1) * o.scale_row_stride * sb + (K / blk + 1) * o.scale_kb_stride * sb;
  FM_REQUIRE(o.scale_row_stride >= 0 && o.scale_kb_stride >= 0 && span < (int64_t(1) << 32),
             "grouped gemm: operand %s scales span more than 4 GiB from their group base", name);
  return 0;
}

// ============================================================================
// split-K reduction of the ragged-K partials
// ============================================================================
// ws [splits][E][M][N] fp32 -> out / out2 rows (row < split: out, else out2 at
// row - split), summed in slice order (deterministic), 4 columns per thread.
// Experts that the mask leaves to the other launch are not written.
struct SplitReduceArgs {
  const float* ws;
  int64_t slice, E, M, N;
  int splits;
  const int32_t* mask;
  int mask_want;
  void* out;
  void* out2;
  int64_t out_gs, out2_gs, split, ld;
  int out_f32;
};

__global__ __launch_bounds__(256) void split_reduce_kernel(SplitReduceArgs a) {
  const int64_t n4 = a.N / 4;
  const int64_t total = a.E * a.M * n4;
  for (int64_t v = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; v < total;
       v += int64_t(gridDim.x) * blockDim.x) {
    const int64_t c = (v % n4) * 4;
    const int64_t r = (v / n4) % a.M;
    const int64_t e = v / (n4 * a.M);
    if (a.mask != nullptr && a.mask[e] != a.mask_want) continue;
    const float* src = a.ws + (e * a.M + r) * a.N + c;
    float4 acc = *reinterpret_cast<const float4*>(src);
    for (int s = 1; s < a.splits; ++s) {
      const float4 u = *reinterpret_cast<const float4*>(src + s * a.slice);
      acc.x += u.x;
      acc.y += u.y;
      acc.z += u.z;
      acc.w += u.w;
    }
    const bool second = r >= a.split;
    const int64_t off = e * (second ? a.out2_gs : a.out_gs) + (second ? r - a.split : r) * a.ld + c;
    if (a.out_f32) {
      st_global(static_cast<float*>(second ? a.out2 : a.out) + off, acc);
    } else {
      uint16_t* d = static_cast<uint16_t*>(second ? a.out2 : a.out) + off;
      st_global(d, make_uint2(hw_bf16x2(acc.x, acc.y), hw_bf16x2(acc.z, acc.w)));
    }
  }
}

}  // namespace fm

using namespace fm;

extern "C" {

}  // extern "C"

namespace {

// Checks the ragged-M arguments and fills the launch parameters (`kind`
// without flags; nn: the weights are stored [K][N]).  Returns 0 with
// p.m_tiles == 0 when there is nothing to do.
int ragged_m_params(int kind, int nn, int paired, const FmGemmOperand* tokens, const FmGemmOperand* weights, int64_t m_tiles,
                    const int32_t* tile_expert, const int32_t* offsets, int E, int64_t N, int64_t K,
                    const int32_t* expert_mask, int mask_want, void* out, int out_dtype, int64_t ld_out,
                    GemmParams& p) {
  FM_REQUIRE(tokens && weights && tile_expert && offsets && out, "fm_grouped_gemm_ragged_m: null pointer");
  // K rows per tensor: a [K][N] operand split along K holds split_rows, then K - split_rows, per group
  const int64_t nn_rows = weights->data2 == nullptr || weights->split_rows <= 0 || weights->split_rows >= K
                              ? K
                              : (weights->split_rows > K - weights->split_rows ? weights->split_rows
                                                                               : K - weights->split_rows);
  FM_REQUIRE(!nn || (((kind == GK_FP8_POW2 && K >= 256) || (kind == GK_BF16 && K >= 128)) && E <= 64 &&
                     N % 256 == 0 && weights->ld >= N && weights->group_stride >= nn_rows * weights->ld &&
                     nn_rows * weights->ld * (kind == GK_BF16 ? 2 : 1) < (int64_t(1) << 32)),
             "fm_grouped_gemm_ragged_m: [K][N] weights need the pow2 kind with K >= 256 or BF16 with K >= 128, "
             "E <= 64, N a multiple of 256, a row pitch >= N, a group stride >= K x pitch and K x pitch bytes "
             "below 2^32 (split along K: the larger part's rows for K)");
  if (int rc = check_operand(*tokens, kind, "tokens")) return rc;
  if (int rc = check_operand(*weights, kind, "weights")) return rc;
  FM_REQUIRE(tokens->data2 == nullptr, "fm_grouped_gemm_ragged_m: the token operand cannot be split");
  FM_REQUIRE(weights->data2 == nullptr ||
                 (kind == GK_BF16 && E <= 64 && K >= 128 && weights->split_rows > 0 &&
                  (nn ? weights->split_rows % 64 == 0 && weights->split_rows < K
                      : weights->split_rows % 256 == 0 && weights->split_rows < N)),
             "fm_grouped_gemm_ragged_m: split weights need the BF16 kind, E <= 64, K >= 128 and a split that is "
             "a multiple of 256 inside N ([K][N] weights: of 64 inside K)");
  if (int rc = check_scale_span(*tokens, kind, m_tiles * 128, K, "tokens")) return rc;
  if (int rc = check_scale_span(*weights, kind, N, K, "weights")) return rc;
  FM_REQUIRE(N > 0 && N % 128 == 0, "fm_grouped_gemm_ragged_m: N must be a positive multiple of 128 (got %lld)", (long long)N);
  FM_REQUIRE(K > 0 && K % 128 == 0, "fm_grouped_gemm_ragged_m: K must be a positive multiple of 128 (got %lld)", (long long)K);
  FM_REQUIRE(E >= 1, "fm_grouped_gemm_ragged_m: E must be >= 1");
  FM_REQUIRE(m_tiles >= 0, "fm_grouped_gemm_ragged_m: m_tiles must be >= 0");
  FM_REQUIRE(tokens->ld >= K && (nn || weights->ld >= K), "fm_grouped_gemm_ragged_m: operand pitch < K");
  FM_REQUIRE(nn || weights->group_stride >= K, "fm_grouped_gemm_ragged_m: weight group stride < K");
  FM_REQUIRE(ld_out >= N && ld_out % 4 == 0, "fm_grouped_gemm_ragged_m: output pitch must be >= N and a multiple of 4");
  FM_REQUIRE(out_dtype == FM_DTYPE_BF16 || out_dtype == FM_DTYPE_F32, "fm_grouped_gemm_ragged_m: bad out dtype");
  FM_REQUIRE(kind != GK_FP8_F32 || weights->scale_row_shift == 7,
             "fm_grouped_gemm_ragged_m: fp32-scaled weights must use 128-row scale blocks");
  FM_REQUIRE(!paired || ((kind == GK_FP8_POW2 || (kind == GK_FP8_MX && !nn)) && E <= 64 && K >= 384 &&
                         tokens->ld % 64 == 0 && weights->data2 == nullptr && (nn || weights->ld % 64 == 0)),
             "fm_grouped_gemm_ragged_m: paired-row operands need the pow2 kind (or MX with [N][K] weights), "
             "E <= 64, K >= 384, unsplit weights and row pitches that are multiples of 64");
  p = GemmParams{};
  p.m_tiles = m_tiles;
  if (m_tiles == 0) return 0;
  p.paired = paired;
  p.P = make_operand(*tokens);
  p.Q = make_operand(*weights);
  p.n_i = N;
  p.K = K;
  p.tile_expert = tile_expert;
  p.m_tiles = m_tiles;
  // sum over experts of ceil(tiles_e / 2) <= (m_tiles + E) / 2
  p.j_tiles = (m_tiles + E + 1) / 2;
  p.offsets = offsets;
  p.E = E;
  p.mask = expert_mask;
  p.mask_want = mask_want;
  p.C = out;
  p.ldC = ld_out;
  p.out_f32 = out_dtype == FM_DTYPE_F32;
  p.split = INT64_MAX;
  p.q_nn = nn;
  return 0;
}

}  // namespace

extern "C" {

int fm_grouped_gemm_ragged_m(int kind, const FmGemmOperand* tokens, const FmGemmOperand* weights,
                             int64_t m_tiles, const int32_t* tile_expert, const int32_t* offsets,
                             int E, int64_t N, int64_t K, const int32_t* expert_mask, int mask_want,
                             void* out, int out_dtype, int64_t ld_out, void* stream) {
  const int nn = (kind & FM_GEMM_W_KMAJOR) != 0;
  // paired: 1 tokens (and [N][K] weights) paired, 2 [K][N] weights paired too
  const int paired = (kind & FM_GEMM_PAIRED) == 0 ? 0 : (nn && (kind & FM_GEMM_W_PAIRED) != 0) ? 2 : 1;
  FM_REQUIRE((kind & FM_GEMM_W_PAIRED) == 0 || (nn && paired),
             "fm_grouped_gemm_ragged_m: FM_GEMM_W_PAIRED needs FM_GEMM_PAIRED and FM_GEMM_W_KMAJOR");
  kind &= ~(FM_GEMM_W_KMAJOR | FM_GEMM_PAIRED | FM_GEMM_W_PAIRED);
  GemmParams p;
  if (int rc = ragged_m_params(kind, nn, paired, tokens, weights, m_tiles, tile_expert, offsets, E, N, K, expert_mask,
                               mask_want, out, out_dtype, ld_out, p))
    return rc;
  if (p.m_tiles == 0) return 0;
  return dispatch_gemm<GM_RAGGED_M>(kind, p, static_cast<hipStream_t>(stream));
}

namespace {

// Checks the ragged-K arguments and fills the launch parameters (the public
// entries differ only in the split).
int ragged_k_params(int kind, const FmGemmOperand* a_t, const FmGemmOperand* b_t, const int32_t* offsets, int E,
                    int64_t M, int64_t N, const int32_t* expert_mask, int mask_want, void* out, int64_t out_gs,
                    void* out2, int64_t out2_gs, int64_t split_rows, int out_dtype, int64_t ld_out, GemmParams& p) {
  FM_REQUIRE(a_t && b_t && offsets && out, "fm_grouped_gemm_ragged_k: null pointer");
  FM_REQUIRE(a_t->data2 == nullptr && b_t->data2 == nullptr, "fm_grouped_gemm_ragged_k: operands cannot be split");
  if (int rc = check_operand(*a_t, kind, "a_t")) return rc;
  if (int rc = check_operand(*b_t, kind, "b_t")) return rc;
  // contraction over token columns: at most the row pitch of the operands
  if (int rc = check_scale_span(*a_t, kind, M, a_t->ld, "a_t")) return rc;
  if (int rc = check_scale_span(*b_t, kind, N, b_t->ld, "b_t")) return rc;
  FM_REQUIRE(M > 0 && M % 128 == 0 && N > 0 && N % 128 == 0,
             "fm_grouped_gemm_ragged_k: M and N must be positive multiples of 128 (got %lld x %lld)",
             (long long)M, (long long)N);
  FM_REQUIRE(E >= 1, "fm_grouped_gemm_ragged_k: E must be >= 1");
  FM_REQUIRE(ld_out >= N && ld_out % 4 == 0, "fm_grouped_gemm_ragged_k: output pitch must be >= N and a multiple of 4");
  FM_REQUIRE(out_dtype == FM_DTYPE_BF16 || out_dtype == FM_DTYPE_F32, "fm_grouped_gemm_ragged_k: bad out dtype");
  FM_REQUIRE(split_rows >= M || (out2 != nullptr && split_rows % 128 == 0 && split_rows > 0),
             "fm_grouped_gemm_ragged_k: split output needs out2 and a 128-aligned split");
  p = GemmParams{};
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
  p.splits = 1;
  return 0;
}

}  // namespace

int fm_grouped_gemm_ragged_k(int kind, const FmGemmOperand* a_t, const FmGemmOperand* b_t,
                             const int32_t* offsets, int E, int64_t M, int64_t N,
                             const int32_t* expert_mask, int mask_want, void* out, int64_t out_gs,
                             void* out2, int64_t out2_gs, int64_t split_rows, int out_dtype,
                             int64_t ld_out, void* stream) {
  const int a_fast = (kind & FM_GEMM_A_FAST) != 0;
  const int paired = (kind & FM_GEMM_PAIRED) != 0;
  kind &= ~(FM_GEMM_A_FAST | FM_GEMM_PAIRED);
  GemmParams p;
  if (int rc = ragged_k_params(kind, a_t, b_t, offsets, E, M, N, expert_mask, mask_want, out, out_gs, out2,
                               out2_gs, split_rows, out_dtype, ld_out, p))
    return rc;
  if (paired) {
    FM_REQUIRE((kind == GK_FP8_POW2 || kind == GK_FP8_MX) && expert_mask == nullptr && E <= 64 &&
                   a_t->ld % 64 == 0 && b_t->ld % 64 == 0 &&
                   int64_t(E) * ((M + 255) / 256) * ((N + 255) / 256) < (int64_t(1) << 28),
               "fm_grouped_gemm_ragged_k: paired-row operands need the pow2 or MX kind, no expert mask, E <= 64, "
               "pitches that are multiples of 64 and fewer than 2^28 tiles");
    p.paired = 1;
  }
  p.rk_jfast = a_fast;
  return dispatch_gemm<GM_RAGGED_K>(kind, p, static_cast<hipStream_t>(stream));
}

int fm_grouped_gemm_ragged_m_k(int kind, const FmGemmOperand* tokens, const FmGemmOperand* weights,
                               int64_t m_tiles, const int32_t* tile_expert, int64_t N, int64_t K, void* out,
                               int out_dtype, int64_t ld_out, const FmGemmOperand* a_t, const FmGemmOperand* b_t,
                               int64_t M2, int64_t N2, void* out2, int64_t out2_gs, void* out2b, int64_t out2b_gs,
                               int64_t split_rows, int out2_dtype, int64_t ld_out2, const int32_t* offsets, int E,
                               const int32_t* expert_mask, int mask_want, void* stream) {
  const int nn = (kind & FM_GEMM_W_KMAJOR) != 0;
  const int a_fast = (kind & FM_GEMM_A_FAST) != 0;
  const int paired = (kind & FM_GEMM_PAIRED) != 0;
  kind &= ~(FM_GEMM_W_KMAJOR | FM_GEMM_A_FAST | FM_GEMM_PAIRED);
  GemmParams pm, pk;
  if (int rc = ragged_m_params(kind, nn, paired, tokens, weights, m_tiles, tile_expert, offsets, E, N, K, expert_mask,
                               mask_want, out, out_dtype, ld_out, pm))
    return rc;
  if (int rc = ragged_k_params(kind, a_t, b_t, offsets, E, M2, N2, expert_mask, mask_want, out2, out2_gs, out2b,
                               out2b_gs, split_rows, out2_dtype, ld_out2, pk))
    return rc;
  pk.rk_jfast = a_fast;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (paired) {
    // every operand paired: one ring walk over the dgrad tiles, then the weight-gradient tiles
    FM_REQUIRE(!nn && expert_mask == nullptr && a_t->ld % 64 == 0 && b_t->ld % 64 == 0 &&
                   int64_t(E) * ((M2 + 255) / 256) * ((N2 + 255) / 256) < (int64_t(1) << 28),
               "fm_grouped_gemm_ragged_m_k: paired-row operands need [N][K] weights, no expert mask, "
               "pitches that are multiples of 64 and fewer than 2^28 weight-gradient tiles");
    pk.paired = 1;
    if (kind != GK_FP8_POW2) {   // MX: the two ring launches (one grid would need both MX scale layouts)
      if (pm.m_tiles > 0)
        if (int rc = dispatch_gemm<GM_RAGGED_M>(kind, pm, s)) return rc;
      return dispatch_gemm<GM_RAGGED_K>(kind, pk, s);
    }
    if (int rc = prepare_gemm<GM_RAGGED_M>(kind, pm)) return rc;
    if (int rc = prepare_gemm<GM_RAGGED_K>(kind, pk)) return rc;
    const int64_t nbm = pm.m_tiles == 0 ? 0 : (pm.n_tiles + 7) / 8 * 8, nbk = (pk.n_tiles + 7) / 8 * 8;
    if (nbm + nbk == 0) return 0;
    const int64_t slots = int64_t(device_cus() / 8 > 0 ? device_cus() / 8 : 1) * 8;
    const dim3 pgrid(unsigned(nbm + nbk < slots ? nbm + nbk : slots)), pblock(512);
    if (nbm == 0) hipLaunchKernelGGL((gemm256r_kernel<GK_FP8_POW2, 0, false, true, false, true>), pgrid, pblock, 0, s, pk, pk);
    else hipLaunchKernelGGL((gemm256r_kernel<GK_FP8_POW2, 0, true, true, false, true>), pgrid, pblock, 0, s, pm, pk);
    return check_launch("fm_grouped_gemm_ragged_m_k");
  }
  if (nn || pm.m_tiles == 0 || (kind != GK_BF16 && kind != GK_FP8_POW2) || !gemm_mk_one_grid()) {
    if (pm.m_tiles > 0)
      if (int rc = dispatch_gemm<GM_RAGGED_M>(kind, pm, s)) return rc;
    return dispatch_gemm<GM_RAGGED_K>(kind, pk, s);
  }
  const GemmParams pm_args = pm, pk_args = pk;   // as the single-launch entries receive them
  if (int rc = prepare_gemm<GM_RAGGED_M>(kind, pm)) return rc;
  if (int rc = prepare_gemm<GM_RAGGED_K>(kind, pk)) return rc;
  const int64_t nbm = (pm.n_tiles + 7) / 8 * 8, nbk = (pk.n_tiles + 7) / 8 * 8;
  if (nbm + nbk == 0) return 0;
  if (expert_mask == nullptr && E <= 64 && pm.K / (kind == GK_BF16 ? 64 : 128) >= 2 &&
      pk.n_tiles < (int64_t(1) << 28) && gemm_persistent_k()) {
    // persistent: one workgroup per CU (a multiple of 8), at most one per tile
    const int64_t slots = int64_t(device_cus() / 8 > 0 ? device_cus() / 8 : 1) * 8;
    const dim3 pgrid(unsigned(nbm + nbk < slots ? nbm + nbk : slots)), pblock(512);
    if (kind == GK_BF16) hipLaunchKernelGGL((gemm256pmk_kernel<GK_BF16>), pgrid, pblock, 0, s, pm, pk);
    else hipLaunchKernelGGL((gemm256pmk_kernel<GK_FP8_POW2>), pgrid, pblock, 0, s, pm, pk);
    return check_launch("fm_grouped_gemm_ragged_m_k");
  }
  if (pm.Q.split != INT64_MAX) {   // split weights: only the persistent ragged-M kernel reads them
    if (int rc = dispatch_gemm<GM_RAGGED_M>(kind, pm_args, s)) return rc;
    return dispatch_gemm<GM_RAGGED_K>(kind, pk_args, s);
  }
  const dim3 grid(unsigned(nbm + nbk)), block(512);
  if (kind == GK_BF16) hipLaunchKernelGGL((gemm256_mk_kernel<GK_BF16>), grid, block, 0, s, pm, pk, nbm);
  else hipLaunchKernelGGL((gemm256_mk_kernel<GK_FP8_POW2>), grid, block, 0, s, pm, pk, nbm);
  return check_launch("fm_grouped_gemm_ragged_m_k");
}

int64_t fm_grouped_gemm_ragged_k_split_workspace_bytes(int E, int64_t M, int64_t N, int splits) {
  if (E < 1 || M < 0 || N < 0 || splits < 1) return -1;
  return int64_t(splits) * E * M * N * int64_t(sizeof(float));
}

int fm_grouped_gemm_ragged_k_split(int kind, const FmGemmOperand* a_t, const FmGemmOperand* b_t,
                                   const int32_t* offsets, int E, int64_t M, int64_t N,
                                   const int32_t* expert_mask, int mask_want, void* out, int64_t out_gs,
                                   void* out2, int64_t out2_gs, int64_t split_rows, int out_dtype,
                                   int64_t ld_out, int splits, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  const int a_fast = (kind & FM_GEMM_A_FAST) != 0;
  kind &= ~FM_GEMM_A_FAST;
  GemmParams p;
  if (int rc = ragged_k_params(kind, a_t, b_t, offsets, E, M, N, expert_mask, mask_want, out, out_gs, out2,
                               out2_gs, split_rows, out_dtype, ld_out, p))
    return rc;
  p.rk_jfast = a_fast;
  FM_REQUIRE(splits >= 1 && splits <= 16, "fm_grouped_gemm_ragged_k_split: splits must be in [1, 16] (got %d)",
             splits);
  FM_REQUIRE(kind != GK_FP8_F32 || splits == 1,
             "fm_grouped_gemm_ragged_k_split: the fp32-scale blockwise kind takes no K split");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (splits == 1) return dispatch_gemm<GM_RAGGED_K>(kind, p, s);
  const int64_t need = fm_grouped_gemm_ragged_k_split_workspace_bytes(E, M, N, splits);
  FM_REQUIRE(workspace != nullptr && workspace_bytes >= need,
             "fm_grouped_gemm_ragged_k_split: workspace of %lld bytes needed, %lld given", (long long)need,
             (long long)workspace_bytes);
  FM_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15) == 0,
             "fm_grouped_gemm_ragged_k_split: workspace must be 16-byte aligned");
  SplitReduceArgs r{};
  r.ws = static_cast<const float*>(workspace);
  r.slice = int64_t(E) * M * N;
  r.E = E;
  r.M = M;
  r.N = N;
  r.splits = splits;
  r.mask = expert_mask;
  r.mask_want = mask_want;
  r.out = p.C;
  r.out2 = p.C2;
  r.out_gs = p.c_gs;
  r.out2_gs = p.c2_gs;
  r.split = p.split;
  r.ld = p.ldC;
  r.out_f32 = p.out_f32;
  // the GEMM writes fp32 partials [splits][E][M][N] into the workspace
  p.C = workspace;
  p.C2 = nullptr;
  p.ldC = N;
  p.c_gs = M * N;
  p.split = INT64_MAX;
  p.out_f32 = 1;
  p.splits = splits;
  p.ws_slice = r.slice;
  if (int rc = dispatch_gemm<GM_RAGGED_K>(kind, p, s)) return rc;
  const int64_t total = int64_t(E) * M * (N / 4);
  const int64_t blocks = (total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192;
  hipLaunchKernelGGL(split_reduce_kernel, dim3(unsigned(blocks)), dim3(256), 0, s, r);
  return check_launch("grouped gemm split-K reduction");
}

}  // extern "C"
