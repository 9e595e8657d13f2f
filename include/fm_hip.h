/* fm_hip.h -- C ABI of libfm_hip.so, the MI355X (gfx950) kernels behind the
 * fp8_flow_moe operator path.
 *
 * The reference exposes this path only as Python names re-exported by
 * nanopsyche (reference fp8/__init__.py:8-24, fp8/flow_moe.py:3-15,
 * fp8/recipes.py:3-7) from the absent `fp8_flow_moe` package, and as the
 * object call made by MoEBase (reference model/moe.py:1313-1332 construct,
 * :1516-1517 and :1557-1558 call).  Each entry point below names the
 * reference function or op sequence it replaces.
 *
 * Conventions
 *   - Plain device pointers, element counts and pitches (in elements), and a
 *     hipStream_t passed as void*.  No allocation, no host synchronisation:
 *     every call only enqueues work on `stream`.
 *   - Return 0 on success; nonzero on a rejected argument or launch failure,
 *     with the message available from fm_last_error_string() (thread-local).
 *   - bf16 is passed as raw 16-bit words, e4m3 (OCP e4m3fn) and e8m0 as bytes.
 *   - Block-scale spec: scale = max(amax, 1e-12) / 448 in fp32 (power-of-two
 *     kinds round it up to 2^ceil(log2)); q = e4m3(clamp(x / scale, +-448)).
 *     MX: code = clamp(exponent(amax) - 8, 0, 254), q = sat_e4m3(x * 2^(127-code)).
 */
#ifndef FM_HIP_H_
#define FM_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
#define FM_DTYPE_BF16 0
#define FM_DTYPE_F32 1

/* quantisation kinds (payload + scale format) */
#define FM_QUANT_BF16 0   /* no quantisation: bf16 payload, no scales          */
#define FM_QUANT_BLOCK 1  /* e4m3, fp32 scale per 128 block                     */
#define FM_QUANT_POW2 2   /* e4m3, power-of-two fp32 scale per 128 block        */
#define FM_QUANT_MX 3     /* e4m3, e8m0 scale per 32 block (OCP MXFP8)          */
/* OR-ed into the kind of fm_quantize / fm_permute / fm_swiglu_quantize /
 * fm_swiglu_backward: the row scales are stored block-major, s[block * ld_s +
 * row] (ld_s >= rows), instead of s[row * ld_s + block].  A grouped-GEMM K step
 * then reads the scales of 256 consecutive rows from one contiguous 1 KiB
 * span (FmGemmOperand scale_row_stride 1, scale_kb_stride ld_s). */
#define FM_SCALES_KMAJOR 0x100
/* OR-ed into the kind (e4m3 kinds) of fm_quantize / fm_quantize_pair /
 * fm_permute / fm_swiglu_quantize / fm_swiglu_backward and into
 * FmWeightJob.kind: the row-major payload q is written in the paired-row
 * layout -- rows 2p and 2p + 1 interleaved in 64-byte pieces, byte (r, c) at
 * q[(r >> 1) * 2 * ld_q + (c >> 6) * 128 + (r & 1) * 64 + (c & 63)] (ld_q a
 * multiple of 64, an even number of rows) -- the operand layout of
 * fm_grouped_gemm_ragged_m with FM_GEMM_PAIRED.  Scales and the transposed
 * output are unchanged. */
#define FM_ROWS_PAIRED 0x400
/* Likewise for the transposed payload qt (its rows are the source columns,
 * an even count): the layout of the weight-gradient operands of
 * fm_grouped_gemm_ragged_k / _m_k with FM_GEMM_PAIRED. */
#define FM_COLS_PAIRED 0x800

/* grouped GEMM arithmetic kinds */
#define FM_GEMM_BF16 0
#define FM_GEMM_FP8_F32 1  /* fp32 block scales, promoted per 128-deep K block */
#define FM_GEMM_FP8_POW2 2 /* power-of-two scales through the scaled MFMA      */
#define FM_GEMM_FP8_MX 3   /* e8m0 per-32 scales through the scaled MFMA       */
/* OR-ed into the kind of fm_grouped_gemm_ragged_k(_split): the output tiles of
 * an expert are walked with a_t's tiles varying fastest (by default b_t's).
 * The workgroups running at one time then cover all of that operand's tiles,
 * which are fetched from memory in the first round only, so pass it when a_t is
 * the operand not in cache (written long before the launch) and b_t the one
 * just written.  The results do not depend on it. */
#define FM_GEMM_A_FAST 0x100
/* OR-ed into the kind of fm_grouped_gemm_ragged_m: the weights are stored
 * [K][N] -- element (n, k) of expert e at data[e * group_stride + k * ld + n]
 * (ld >= N), e.g. an expert's w2 [H, D] rows for the down projection -- and
 * read transposed in LDS, so no [N][K] copy is needed.  FM_GEMM_FP8_POW2 with
 * 128 x 128 weight blocks (scale of rows n, K block kb at
 * s[e * scale_group_stride + (n >> 7) * scale_row_stride + kb * scale_kb_stride])
 * and K >= 256, or FM_GEMM_BF16 with K >= 128; E <= 64, N a multiple of 256,
 * K x ld bytes below 2^32.  The results are those of the [N][K] layout bit for
 * bit. */
#define FM_GEMM_W_KMAJOR 0x200
/* OR-ed into the kind of fm_grouped_gemm_ragged_m (FM_GEMM_FP8_POW2, E <= 64,
 * K >= 384, row pitches multiples of 64): the token operand, and the weights
 * unless FM_GEMM_W_KMAJOR, are in the paired-row layout -- rows 2p and 2p + 1
 * interleaved in 64-byte pieces, byte (r, k) at
 * (r >> 1) * 2 * ld + (k >> 6) * 128 + (r & 1) * 64 + (k & 63) -- which the
 * persistent kernel streams in 64-deep half steps through a four-slot ring.
 * The results are those of the row-major operands bit for bit.  FM_ROWS_PAIRED
 * makes the quantisers write this layout. */
#define FM_GEMM_PAIRED 0x400
/* With FM_GEMM_W_KMAJOR: the [K][N] weights are in the paired-row layout too
 * (K rows 2p and 2p + 1 interleaved in 64-byte pieces of N), e.g. the paired
 * gate|up operand read as [K = 2H][N = D] for the input gradient. */
#define FM_GEMM_W_PAIRED 0x800

/* gating functions (reference model/moe.py:44-46 GatingFunction) */
#define FM_GATING_SOFTMAX 0
#define FM_GATING_SIGMOID 1

/* ------------------------------------------------------------ library ---- */
const char* fm_last_error_string(void);
const char* fm_version(void);
/* Hash of the sources the library was built from (csrc/ and include/), set
 * by the build; the Python loader refuses a library whose hash differs from
 * the sources beside it (a stale build). */
const char* fm_source_hash(void);
/* Host-side codec (no GPU): the same f32 -> e4m3 routine the kernels use,
 * exported so tests can check it against other implementations. */
void fm_host_encode_e4m3(const float* in, uint8_t* out, int64_t n);
void fm_host_decode_e4m3(const uint8_t* in, float* out, int64_t n);
/* HBM bandwidth probe (no counterpart in the reference: the measurement the
 * HBM-bound kernels are compared against).  kind 0: copy `bytes` from src to
 * dst, one 4 KiB chunk per workgroup; 1: read src (dst: a 1 KiB sink);
 * 2: write dst.  bytes a positive multiple of 4096, 16-byte aligned buffers. */
int fm_hbm_probe(int kind, const void* src, void* dst, int64_t bytes, void* stream);
/* Device conversion check: x [n] fp32 (n % 4 == 0) encoded to e4m3 (after a
 * clamp to +-448) and to bf16 by the gfx950 convert instructions (*_hw) and by
 * the integer routines (*_sw).  The kernels use the hardware path; a GPU test
 * asserts the two agree bit for bit. */
int fm_convert_check(const float* x, int64_t n, void* e4m3_hw, void* e4m3_sw, void* bf16_hw,
                     void* bf16_sw, void* stream);
/* Device decode check: e4m3 codes [n] (n % 4 == 0) decoded to fp32 by the
 * gfx950 convert instruction (hw, used by the scaling-aware transpose) and by
 * the integer routine (sw). */
int fm_decode_check(const void* codes, int64_t n, float* hw, float* sw, void* stream);

/* ------------------------------------------------------- quantisation ---- */
/* Replaces fp8_flow_moe.quantize_to_fp8 for activations (1x128 / MX 1x32 row
 * blocks), fused with the 128x1 / 32x1 column-block quantisation of the
 * transpose when qt != NULL (reference fp8/__init__.py:14; "no double
 * quantisation", train/README.md:99-100).  x [rows, cols] bf16 or fp32.
 * Row output q [rows, cols] + s [rows, cols/128] fp32 (or [rows, cols/32] e8m0);
 * transposed output qt [cols, rows] + st [rows/128, cols] (or [rows/32, cols]).
 * kind FM_QUANT_POW2: the transposed output is the scaling-aware transpose
 * of the row output.  FM_QUANT_BF16: plain bf16 copy / transpose. */
int fm_quantize(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ld_x, int kind,
                void* q, int64_t ld_q, void* s, int64_t ld_s, void* qt, int64_t ld_qt, void* st,
                int64_t ld_st, void* stream);

/* fm_quantize of the fused gate|up weight without materialising it: a and b
 * are [groups, rows, cols] stacks (w1 and w3 of model/moe.py:1293-1295,
 * groups = experts, rows = H; pitch ld, dtype bf16 or fp32) read as one
 * [groups * 2 * rows, cols] matrix whose group g holds a's rows then b's
 * (torch.cat([w1_e, w3_e]) per expert).  Outputs and kinds as fm_quantize (the
 * MX recipe quantises expert weights this way: 1x32 along cols, 32x1 along
 * the stacked rows). */
int fm_quantize_pair(const void* a, const void* b, int dtype, int64_t groups, int64_t rows,
                     int64_t cols, int64_t ld, int kind, void* q, int64_t ld_q, void* s, int64_t ld_s,
                     void* qt, int64_t ld_qt, void* st, int64_t ld_st, void* stream);

/* Replaces quantize_to_fp8 for expert weights (128x128 blocks), batched over
 * `groups` matrices [rows, cols] of w (pitch ld_w, group stride gs_w), writing
 * into row offset q_row_off of q (and column offset qt_col_off of the
 * transposed payload qt, same blocks), so w1 and w3 can be packed into one
 * [E, 2H, D] operand.  kind: FM_QUANT_BF16 / BLOCK / POW2. */
int fm_quantize_weight(const void* w, int w_dtype, int64_t groups, int64_t rows, int64_t cols,
                       int64_t ld_w, int64_t gs_w, int kind, void* q, int64_t ld_q, int64_t gs_q,
                       int64_t q_row_off, float* s, int64_t ld_s, int64_t gs_s, void* qt,
                       int64_t ld_qt, int64_t gs_qt, int64_t qt_col_off, float* st, int64_t ld_st,
                       int64_t gs_st, void* stream);

/* One fm_quantize_weight job (same arguments). */
typedef struct FmWeightJob {
  const void* w;
  int w_dtype;
  int64_t groups, rows, cols, ld_w, gs_w;
  int kind;
  void* q;
  int64_t ld_q, gs_q, q_row_off;
  float* s;
  int64_t ld_s, gs_s;
  void* qt;
  int64_t ld_qt, gs_qt, qt_col_off;
  float* st;
  int64_t ld_st, gs_st;
} FmWeightJob;

/* Same replacement as fm_quantize_weight (quantize_to_fp8 for expert weights,
 * reference fp8/__init__.py:14): up to 4 jobs with equal groups, rows, cols and
 * w_dtype in one launch (w1, w3 and w2 of one recipe), so the block tails of
 * separate launches do not add up. */
int fm_quantize_weight_batch(const FmWeightJob* jobs, int n_jobs, void* stream);

/* Replaces fp8_flow_moe.dequantize_from_fp8 (reference fp8/__init__.py:15).
 * out[r][c] = decode(q[r][c]) * S, S = s[(r >> row_shift) * s_row_stride +
 * (c >> col_shift) * s_col_stride] (fp32, or e8m0 when s_e8m0). */
int fm_dequantize(const void* q, int64_t rows, int64_t cols, int64_t ld_q, const void* s,
                  int s_e8m0, int row_shift, int col_shift, int64_t s_row_stride,
                  int64_t s_col_stride, void* out, int out_dtype, int64_t ld_out, void* stream);

/* Replaces fp8_flow_moe.scaling_aware_transpose (reference fp8/__init__.py:16):
 * row-quantised q [rows, cols] + s [rows, cols/128] -> column-quantised
 * transpose qt [cols, rows] + st [rows/128, cols] without the bf16 source.
 * st = largest row scale in the 128x128 tile; exact for power-of-two scales
 * outside the e4m3 subnormal range. */
int fm_scaling_aware_transpose(const void* q, int64_t rows, int64_t cols, int64_t ld_q,
                               const float* s, int64_t ld_s, void* qt, int64_t ld_qt, float* st,
                               int64_t ld_st, void* stream);

/* ------------------------------------------------------------ routing ---- */
/* Replaces MoERouter._softmax_gating / _sigmoid_gating /
 * _routing_replay_gating and the l2 weight normalisation of MoERouter.forward
 * (reference model/moe.py:158-170, :187-265): per token, top-K of the logits
 * (softmax: weights = softmax over the K selected logits) or of
 * sigmoid(logits) (weights / (sum + 1e-8)).  Selection order: NaN above
 * every number (as torch.topk), then larger, then the lower expert index; an
 * expert is selected at most once.  replay_indices [T, K] (int64 or int32,
 * or NULL): R3 routing replay -- weights = softmax(all logits) restricted to
 * the replayed experts and renormalised (sum clamped to >= 1e-8), the K
 * largest in order, whatever `gating` is.  flags: FM_GATING_L2_NORMALIZE
 * divides the K weights by their l2 norm + 1e-8.  E <= 256,
 * K <= min(E, 64).  prob_partial [n_waves, E] (or NULL) receives per-wave sums
 * of the full softmax, z_partial [n_waves] (or NULL) per-wave sums of
 * logsumexp(logits)^2, both for fm_aux_loss.  n_waves: positive multiple of 4
 * (grid size). */
#define FM_GATING_L2_NORMALIZE 1
int fm_topk_gating(const float* logits, int64_t T, int E, int64_t ld, int K, int gating, int flags,
                   const void* replay_indices, int replay_i64, float* weights, void* indices, int indices_i64,
                   float* prob_partial, float* z_partial, int64_t n_waves, void* stream);

/* Replaces MoERouter._load_balancing_loss and the z-loss term (reference
 * model/moe.py:172-178, :267-281):
 * loss[0] = E * sum_e (counts[e] / T) * (sum_w prob_partial[w][e] / T)
 *           + z_loss_multiplier * sum_w z_partial[w] / T   (z_partial may be NULL). */
int fm_aux_loss(const float* prob_partial, int64_t n_waves, const int32_t* counts, int E, int64_t T,
                const float* z_partial, float z_loss_multiplier, float* loss, void* stream);

/* Replaces the gate of MoERouter.forward (reference model/moe.py:151-154):
 * logits[t][e] = sum_d x[t][d] w[e][d] + bias[e] + score_bias[e] in fp32, the
 * reference's gate(x.float()) (nn.Linear(D, E, bias=True), :107) plus the
 * DeepSeek-V3 score bias.  x bf16 or fp32 [T, D] (pitch ld_x), w fp32 or bf16
 * (w_dtype) [E, D] (pitch ld_w, a multiple of 4), bias [E] in w's dtype or
 * null, score_bias fp32 [E] or null.  E <= 256, D % 8 == 0. */
int fm_router_logits(const void* x, int x_dtype, int64_t ld_x, int64_t T, int64_t D, const void* w, int w_dtype,
                     int64_t ld_w, const void* bias, const float* score_bias, int E, float* logits, int64_t ld_l,
                     void* stream);

/* Replaces MoERouter.forward (reference model/moe.py:133-184, jitter aside)
 * with its load-balancing loss (:267-281) and expert-count update
 * (:284-292): the gate as fm_router_logits (logits written, score bias
 * included), the gating as fm_topk_gating (gating, flags, replay), counts[E]
 * of the T*K slots (added to tokens_per_expert / total_tokens when given, as
 * fm_expert_counts with tokens = T) and loss = E * sum_e f_e P_e (+ z-loss
 * with z_loss_multiplier != 0) as fm_aux_loss.  For E <= 8 and D a multiple
 * of 512 with the gate [8, D] in 64 KiB (D <= 2048 for an fp32 gate, <= 4096
 * for a bf16 one) the gate, gating, loss partials and counts run as one pass
 * over x plus one small kernel (fm_router_forward_fused says which); other
 * shapes launch the steps separately.  T > 0; the workspace holds
 * fm_router_forward_workspace_bytes(T, E) bytes. */
int64_t fm_router_forward_workspace_bytes(int64_t T, int E);
int fm_router_forward_fused(int E, int64_t D, int w_dtype);
int fm_router_forward(const void* x, int x_dtype, int64_t ld_x, int64_t T, int64_t D, const void* w, int w_dtype,
                      int64_t ld_w, const void* bias, const float* score_bias, int E, int K, int gating, int flags,
                      const void* replay_indices, int replay_i64, float* logits, int64_t ld_l, float* weights,
                      void* indices, int indices_i64, int32_t* counts, int64_t* tokens_per_expert,
                      int64_t* total_tokens, float z_loss_multiplier, float* loss, void* workspace,
                      int64_t workspace_bytes, void* stream);

/* counts[e] = number of the n routed slots with index e (the f_i numerator of
 * MoERouter._load_balancing_loss, model/moe.py:271-274); indices outside
 * [0, E) are not counted.  E <= 1024.  With tokens_per_expert [E] and
 * total_tokens [1] (int64, both or neither) the counts are also added to those
 * running totals and `tokens` (the number of routed tokens) to total_tokens:
 * MoERouter._update_expert_counts (:284-292), which adds per-expert slot
 * counts and indices.shape[0] * indices.shape[1] = B * S tokens for its
 * [B, S, K] indices, kept on the device. */
int fm_expert_counts(const void* indices, int indices_i64, int64_t n, int E, int32_t* counts,
                     int64_t* tokens_per_expert, int64_t* total_tokens, int64_t tokens, void* stream);

/* Replaces MoERouter.post_batch on one GPU (reference model/moe.py:294-321,
 * the DeepSeek-V3 score-bias update): if total_tokens != 0,
 * score_bias[e] += gamma * (tokens_per_expert[e] / total_tokens - 1 / E) in
 * fp32 and both running totals are set to 0; otherwise nothing changes.  The
 * reference's sign is kept (an expert above its share gets a larger bias).
 * With expert parallelism the caller all-reduces the two totals first, as
 * the reference does (:303-305). */
int fm_score_bias_update(int64_t* tokens_per_expert, int64_t* total_tokens, int E, float gamma, float* score_bias,
                         void* stream);

/* Backward of the gating, the weight normalisation, the load-balancing loss
 * and the z-loss (reference model/moe.py:158-184, :187-281 under autograd):
 * dlogits [T, E] from the gradient of the top-k weights (dweights [T, K], or
 * null) and of the aux loss (daux: device scalar, or null; needs counts [E]
 * of the forward routing).  gating: FM_GATING_SOFTMAX (softmax over the K
 * selected logits) or FM_GATING_SIGMOID (sigmoid scores / (sum + 1e-8));
 * replay != 0: the forward replayed `indices` (R3: softmax over them, for
 * either gating).  flags: FM_GATING_L2_NORMALIZE as the forward used it.
 * z_loss_multiplier: 0 when the loss had no z-loss term.  logits as the
 * forward used them (score bias included). */
int fm_gating_grad(const float* logits, int64_t T, int E, int64_t ld_l, int K, int gating, int flags,
                   int replay, const void* indices, int indices_i64, const float* dweights, const float* daux,
                   const int32_t* counts, float z_loss_multiplier, float* dlogits, int64_t ld_d, void* stream);

/* fm_gating_grad with the weights' gradient formed in the same pass instead
 * of read (reference MoEBase.forward's output = sum_k w[t,k] y[row(t,k)]
 * under autograd, model/moe.py:1594, and the gating of :158-184):
 * dweights[t][k] = <dout[t], y[row_of[t K + k]]> in fp32 (0 for a slot with
 * row -1), dout bf16 [T, D] (pitch ld_do), y bf16 expert outputs (pitch ld_y);
 * K <= 8.  dweights_out [T, K] receives it when not null.  With dout null it
 * is fm_gating_grad. */
int fm_gating_grad_dot(const float* logits, int64_t T, int E, int64_t ld_l, int K, int gating, int flags, int replay,
                       const void* indices, int indices_i64, const float* dweights, const void* dout, int64_t ld_do,
                       const void* y, int64_t ld_y, const int32_t* row_of, int64_t D, float* dweights_out,
                       const float* daux, const int32_t* counts, float z_loss_multiplier, float* dlogits,
                       int64_t ld_d, void* stream);

/* Backward of the gate (reference nn.Linear of model/moe.py:107 under
 * autograd): dx = dlogits w (x's dtype, null to skip; w fp32 or bf16),
 * dw = dlogits^T x and db = sum_t dlogits (fp32 sums, null to skip, written
 * as dw_dtype / db_dtype), summed in a fixed order; dw and db need a
 * workspace of fm_router_workspace_bytes(T, D, E) bytes. */
int64_t fm_router_workspace_bytes(int64_t T, int64_t D, int E);
int fm_router_backward(const float* dlogits, int64_t ld_dl, const void* x, int x_dtype, int64_t ld_x, int64_t T,
                       int64_t D, const void* w, int w_dtype, int64_t ld_w, int E, void* dx, int64_t ld_dx, void* dw,
                       int dw_dtype, int64_t ld_dw, void* db, int db_dtype, void* workspace, int64_t workspace_bytes,
                       void* stream);

/* Replaces RMSNorm.forward (reference model/norm.py:32-49, full_precision) as
 * MoEHybridTransformerBlock applies it before the MoE (model/transformer.py:
 * 261-263), fused with the activation quantisation: r = 1 / sqrt(mean(x^2) +
 * eps) and y = (x r) w per row in fp32.  x bf16 or fp32 [T, D] (pitch ld_x),
 * w bf16 or fp32 [D]; D = 512 n, n in 1..8, 10, 12, 14, 16.  Outputs, each
 * optional: y as bf16 [T, D] (pitch ld_y); the e4m3 row blocks of that bf16 y
 * (kind FM_QUANT_BLOCK / _POW2: fp32 scale per 128 columns, s [T, ld_s];
 * FM_QUANT_MX: e8m0 per 32 columns; kind -1: none); rstd [T] (r, for the
 * backward).  One read of x. */
int fm_rmsnorm_quantize(const void* x, int x_dtype, int64_t ld_x, int64_t T, int64_t D, const void* w, int w_dtype,
                        float eps, void* y, int64_t ld_y, int kind, void* q, int64_t ld_q, void* s, int64_t ld_s,
                        float* rstd, void* stream);

/* Backward of RMSNorm (reference model/norm.py:32-49 under autograd): with
 * g = dy w, dx = r g - (r^3 / D) (sum_j g_j x_j) x in x's dtype, and
 * dw = sum_t dy x r (fp32 sums, written as dw_dtype; null to skip), summed in
 * a fixed order through a workspace of fm_rmsnorm_backward_workspace_bytes(T,
 * D) bytes.  dy in x's dtype; rstd as fm_rmsnorm_quantize wrote it. */
int64_t fm_rmsnorm_backward_workspace_bytes(int64_t T, int64_t D);
int fm_rmsnorm_backward(const void* dy, int64_t ld_dy, const void* x, int x_dtype, int64_t ld_x, int64_t T, int64_t D,
                        const void* w, int w_dtype, const float* rstd, void* dx, int64_t ld_dx, void* dw,
                        int dw_dtype, void* workspace, int64_t workspace_bytes, void* stream);

/* Sizes for fm_route_sort: padded-buffer row bound 128 * max(1, floor((A +
 * 127 E) / 128)) (every group padded to 128 rows fits; one group: exactly
 * the padded rows), and workspace bytes. */
int64_t fm_route_rows_max(int64_t assignments, int E);
int64_t fm_route_workspace_bytes(int64_t assignments, int E);

/* Replaces the per-expert `(indices == e).any(-1).nonzero()` token lists of
 * MoEBase._compute_experts_padded_bmm (reference model/moe.py:1565-1567) and
 * the routing half of fp8_flow_moe.fused_permute_pad (fp8/__init__.py:19):
 * stable counting sort of the T*K assignments a = t*K + k by expert.
 * counts [E], offsets [E+1] (padded to multiples of 128), row_of [T*K]
 * (-1 for indices outside [0, E), which the reference loop also ignores),
 * assign_of_row [rows_max] (-1 on pad rows), tile_expert [rows_max/128]
 * (-1 past the last group), use_fp8 [E] (counts[e] >= threshold; may be NULL). */
int fm_route_sort(const void* indices, int indices_i64, int64_t T, int K, int E,
                  int64_t threshold, int32_t* counts, int32_t* offsets, int32_t* row_of,
                  int32_t* assign_of_row, int64_t rows_max, int32_t* tile_expert,
                  int32_t* use_fp8, void* workspace, int64_t workspace_bytes, void* stream);

/* For the fp8_gemm_threshold switch (reference model/moe.py:1215-1216,
 * cli.py:55-63): the routing sort's tile_expert [n_tiles] split by precision,
 * tiles_fp8[t] = tile_expert[t] if that expert's use_fp8 flag is set, else -1,
 * and tiles_bf16[t] the converse (-1 where tile_expert is -1).  Passed as the
 * tile_valid list of fm_permute / fm_swiglu_quantize / fm_swiglu_backward,
 * they make each precision's producers write only the rows of the experts
 * whose GEMMs read them. */
int fm_route_tile_masks(const int32_t* tile_expert, int64_t n_tiles, const int32_t* use_fp8, int32_t* tiles_fp8,
                        int32_t* tiles_bf16, void* stream);

/* Replaces the token dropping of MoEBase._apply_capacity (reference
 * model/moe.py:1395-1448): each expert's tokens ranked in token order, a token
 * kept when every one of its valid slots ranks below `capacity`.  Inputs: the
 * indices [T, K] and the counts, offsets and row_of of fm_route_sort on them.
 * Outputs: pos_of [T] (the token's position among the kept tokens, -1 if
 * dropped), kept_index [T] (first n_kept entries: the kept tokens in order),
 * n_kept [1], drops [E] = max(0, counts[e] - capacity) (the reference's
 * per-expert drop counts; their sum is its `dropped`).  workspace: at least
 * fm_capacity_workspace_bytes(T) bytes, no initial contents needed. */
int64_t fm_capacity_workspace_bytes(int64_t T);
int fm_capacity_select(const void* indices, int indices_i64, int64_t T, int K, int E, const int32_t* counts,
                       const int32_t* offsets, const int32_t* row_of, int64_t capacity, int32_t* pos_of,
                       int32_t* kept_index, int32_t* n_kept, int32_t* drops, void* workspace,
                       int64_t workspace_bytes, void* stream);

/* Replaces the row selections around capacity dropping (reference
 * model/moe.py:1445-1447 `x[keep_mask]`, and :1386-1391, the scatter of the
 * kept tokens' outputs into a zero [B*S, D] buffer): dst row i (pitch ld_dst
 * bytes) = src row index[i] (pitch ld_src bytes, n_src rows), zeros where
 * index[i] is outside [0, n_src).  row_bytes and pitches multiples of 4,
 * pointers 4-byte aligned. */
int fm_gather_rows(const void* src, int64_t n_src, int64_t ld_src, const int32_t* index, int64_t n,
                   int64_t row_bytes, void* dst, int64_t ld_dst, void* stream);

/* fm_route_sort, then fm_quantize_weight_batch(jobs, n_jobs) on the same
 * stream, with the outputs of the two calls.  No counterpart in the
 * reference: the sort's launches occupy a few CUs for a few microseconds, so
 * part of the weight batch's 128x128 blocks run as extra workgroups of those
 * launches and the rest as a launch of their own after the sort (the shares
 * change only timing, never the bytes written).  For a layer that refreshes
 * its expert weights in the same forward that routes its tokens.  jobs as
 * fm_quantize_weight_batch takes them (1-4, equal shapes and dtype); their
 * outputs must not alias the sort's. */
int fm_route_sort_weights(const void* indices, int indices_i64, int64_t T, int K, int E, int64_t threshold,
                          int32_t* counts, int32_t* offsets, int32_t* row_of, int32_t* assign_of_row,
                          int64_t rows_max, int32_t* tile_expert, int32_t* use_fp8, void* workspace,
                          int64_t workspace_bytes, const FmWeightJob* jobs, int n_jobs, void* stream);

/* No counterpart in the reference.  fm_route_sort without the workspace
 * argument and without any allocation, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Outputs and their meaning are fm_route_sort's.  The
 * block histogram lives in a fixed device array of
 * fm_route_sort_noalloc_max_workspace_bytes() bytes (2 MiB) per GPU, held
 * until the process ends; a call needing more than that
 * (fm_route_workspace_bytes(T*K, E) larger) is rejected with an error.  All
 * calls on one GPU share that array: calls that overlap on one GPU (other
 * streams or host threads) race; calls ordered on one stream do not. */
int64_t fm_route_sort_noalloc_max_workspace_bytes(void);
int fm_route_sort_noalloc(const void* indices, int indices_i64, int64_t T, int K, int E,
                          int64_t threshold, int32_t* counts, int32_t* offsets, int32_t* row_of,
                          int32_t* assign_of_row, int64_t rows_max, int32_t* tile_expert,
                          int32_t* use_fp8, void* stream);

/* Replaces fp8_flow_moe.fused_permute_pad (reference fp8/__init__.py:19) and
 * the gather + pad of model/moe.py:1571,1577-1580: row r of the padded buffer
 * is x[assign_of_row[r] / K] (times weights[assign_of_row[r]] if weights !=
 * NULL), zeros on pad rows, written as `kind` with optional transposed output
 * (same layout rules as fm_quantize).  tile_valid (optional, e.g. the
 * tile_expert map of fm_route_sort): 128-row tiles t with tile_valid[t] < 0 are
 * not written. */
int fm_permute(const void* x, int64_t T, int64_t D, int64_t ld_x, const int32_t* assign_of_row,
               int64_t rows, int K, const float* weights, int kind, void* q, int64_t ld_q, void* s,
               int64_t ld_s, void* qt, int64_t ld_qt, void* st, int64_t ld_st,
               const int32_t* tile_valid, void* stream);

/* Replaces fp8_flow_moe.fused_unpermute_unpad (reference fp8/__init__.py:20)
 * and the weighted scatter-add of model/moe.py:1594:
 * out[t] = addend[t] + sum_k weights[t*K+k] * y[row_of[t*K+k]] (weights NULL
 * -> 1, addend bf16 [T, D] pitch ld_add or NULL -> 0), fp32 sum in slot order,
 * one rounding to out_dtype.  The addend lets a MoE layer's input gradient
 * take the router's share in the same pass (the sum autograd forms for an
 * input feeding both the router and the experts, model/moe.py:1347-1375).
 * y, out and addend start on 16-byte boundaries; D and the pitches are
 * multiples of 8. */
int fm_unpermute(const void* y, int64_t ld_y, const int32_t* row_of, const float* weights,
                 int64_t T, int K, int64_t D, void* out, int out_dtype, int64_t ld_out,
                 const void* addend, int64_t ld_add, void* stream);

/* fm_unpermute plus the router's share of a MoE layer's input gradient,
 * dx[t] += sum_e dlogits[t][e] * gate_w[e] (the backward of the gate
 * nn.Linear of reference model/moe.py:107, :151 for an input that also feeds
 * the experts), in the same pass: out[t] = addend[t] + sum_k weights[t*K+k]
 * y[row_of[t*K+k]] + sum_e dlogits[t*ld_dl+e] gate_w[e*ld_w + :], fp32 sums in
 * that order (the router's terms as fused multiply-adds), one rounding.
 * E <= 8; gate_w bf16 or fp32 [E, D]; y, out, addend and gate_w start on
 * 16-byte boundaries (dlogits may not). */
int fm_unpermute_router(const void* y, int64_t ld_y, const int32_t* row_of, const float* weights,
                        int64_t T, int K, int64_t D, void* out, int out_dtype, int64_t ld_out,
                        const void* addend, int64_t ld_add, const float* dlogits, int64_t ld_dl,
                        const void* gate_w, int gate_dtype, int64_t ld_w, int E, void* stream);

/* Gradient of the combine with respect to the router weights (autograd of
 * model/moe.py:1594 in the reference): dw[a] = <dout[a/K], y[row_of[a]]>. */
int fm_router_weight_grad(const void* dout, int64_t ld_do, const void* y, int64_t ld_y,
                          const int32_t* row_of, int64_t T, int K, int64_t D, float* dw,
                          void* stream);

/* ------------------------------------------------------------- SwiGLU ---- */
/* Replaces fp8_flow_moe.fused_swiglu_quantize / fused_silu_multiply_quantize
 * (reference fp8/__init__.py:17-18; math of model/moe.py:1590, 1181-1183):
 * h = silu(g) * u from bf16 g, u, emitted as `kind` (fm_quantize layouts). */
int fm_swiglu_quantize(const void* g, int64_t ld_g, const void* u, int64_t ld_u, int64_t rows,
                       int64_t H, int kind, void* q, int64_t ld_q, void* s, int64_t ld_s, void* qt,
                       int64_t ld_qt, void* st, int64_t ld_st, const int32_t* tile_valid,
                       void* stream);

/* Backward of SwiGLU (autograd of model/moe.py:1590 in the reference):
 * [dg | du] with dg = dh*u*s*(1+g*(1-s)), du = dh*g*s, s = sigmoid(g), as a
 * [rows, 2H] operand emitted as `kind` (one read of g, u, dh per element).
 * tile_valid as for fm_permute. */
int fm_swiglu_backward(const void* g, int64_t ld_g, const void* u, int64_t ld_u, const void* dh,
                       int64_t ld_dh, int64_t rows, int64_t H, int kind, void* q, int64_t ld_q,
                       void* s, int64_t ld_s, void* qt, int64_t ld_qt, void* st, int64_t ld_st,
                       const int32_t* tile_valid, void* stream);

/* The fp32 values fm_swiglu_quantize (dh == NULL: h = silu(g) * u, out [rows, H])
 * and fm_swiglu_backward (out [rows, 2H] = [dg | du]) quantise, computed by
 * the same device code and written unrounded -- for checking those fused
 * kernels' arithmetic against the reference's silu (model/moe.py:1181-1183)
 * and their quantisation against a quantiser applied to these values. */
int fm_swiglu_values(const void* g, int64_t ld_g, const void* u, int64_t ld_u, const void* dh, int64_t ld_dh,
                     int64_t rows, int64_t H, float* out, int64_t ld_out, void* stream);

/* ------------------------------------------------------- grouped GEMM ---- */
/* One operand of the grouped GEMM: K-contiguous rows.  Scale of (row, kb) is
 * scale[g*scale_group_stride + (row >> scale_row_shift)*scale_row_stride +
 * kb*scale_kb_stride], kb counting 128-blocks (fp32 / pow2) or 32-blocks (MX).
 * data2 (NULL: unused) splits each group's rows over two tensors of the same
 * pitch and group stride: rows r >= split_rows are row r - split_rows of
 * data2 -- the weights of fm_grouped_gemm_ragged_m read from w1 and w3 as
 * they are stored, without stacking them.  BF16 weights only, at most 64
 * experts; split_rows a multiple of 256 inside N, or, with FM_GEMM_W_KMAJOR
 * (rows are K rows), a multiple of 64 inside K. */
typedef struct FmGemmOperand {
  const void* data;
  int64_t ld;            /* row pitch, elements */
  int64_t group_stride;  /* elements between experts (weights), else 0 */
  const void* scale;     /* fp32, or e8m0 bytes for FM_GEMM_FP8_MX; NULL for bf16 */
  int64_t scale_row_stride;
  int64_t scale_kb_stride;
  int64_t scale_group_stride;
  int scale_row_shift;   /* 7 for 128x128 weight blocks, 0 otherwise */
  const void* data2;     /* rows from split_rows on (NULL: none) */
  int64_t split_rows;
} FmGemmOperand;

/* Replaces fp8_flow_moe.fp8_grouped_gemm (reference fp8/__init__.py:21) and
 * the per-expert torch.bmm calls of model/moe.py:1588-1591 (forward and
 * dgrad): out[r][n] = sum_k tokens[r][k] * weights_e[n][k] for the rows r of
 * expert e, offsets[e] <= r < offsets[e+1] (offsets and tile_expert as written
 * by fm_route_sort: [E+1] padded group starts and the expert of each 128-row
 * tile, -1 past the last group).  Experts with expert_mask[e] != mask_want
 * when expert_mask != NULL are skipped -- the fp8_gemm_threshold switch of
 * model/moe.py:1215-1216.  N, K multiples of 128. */
int fm_grouped_gemm_ragged_m(int kind, const FmGemmOperand* tokens, const FmGemmOperand* weights,
                             int64_t m_tiles, const int32_t* tile_expert, const int32_t* offsets,
                             int E, int64_t N, int64_t K, const int32_t* expert_mask, int mask_want,
                             void* out, int out_dtype, int64_t ld_out, void* stream);

/* Weight-gradient grouped GEMM (autograd of model/moe.py:1588-1591 with
 * respect to w1/w2/w3): out_e[m][n] = sum over the tokens t of expert e
 * (columns offsets[e]..offsets[e+1] of a_t and b_t) of a_t[m][t] * b_t[n][t].
 * Rows m >= split_rows go to out2 (row m - split_rows), so dW1|dW3 land in two
 * tensors.  Experts with no tokens get zeros. */
int fm_grouped_gemm_ragged_k(int kind, const FmGemmOperand* a_t, const FmGemmOperand* b_t,
                             const int32_t* offsets, int E, int64_t M, int64_t N,
                             const int32_t* expert_mask, int mask_want, void* out, int64_t out_gs,
                             void* out2, int64_t out2_gs, int64_t split_rows, int out_dtype,
                             int64_t ld_out, void* stream);

/* fm_grouped_gemm_ragged_m followed by fm_grouped_gemm_ragged_k on the same
 * stream, with the same offsets, E and expert mask, as one grid: for a
 * backward's dgrad dH = dY w2_e (reference model/moe.py:1588-1591, the bmm's
 * input gradient) and the weight gradient dW2 = h^T dY (the bmm's weight
 * gradient), which read the same permuted dY and are independent.  Run back
 * to back each leaves its last round of tiles part-empty; in one grid the
 * weight-gradient tiles fill the dgrad's last round.  The arguments are those
 * of the two entries (M2, N2, out2 ... ld_out2: fm_grouped_gemm_ragged_k's M,
 * N, out ... ld_out); `kind` takes FM_GEMM_A_FAST for the weight gradient and
 * FM_GEMM_W_KMAJOR for the dgrad.  The outputs equal those of the two calls
 * bit for bit.  Kinds other than BF16 and FP8 pow2 (paired MX operands
 * included), and [K][N] weights, run as the two launches. */
int fm_grouped_gemm_ragged_m_k(int kind, const FmGemmOperand* tokens, const FmGemmOperand* weights,
                               int64_t m_tiles, const int32_t* tile_expert, int64_t N, int64_t K, void* out,
                               int out_dtype, int64_t ld_out, const FmGemmOperand* a_t, const FmGemmOperand* b_t,
                               int64_t M2, int64_t N2, void* out2, int64_t out2_gs, void* out2b, int64_t out2b_gs,
                               int64_t split_rows, int out2_dtype, int64_t ld_out2, const int32_t* offsets, int E,
                               const int32_t* expert_mask, int mask_want, void* stream);

/* fm_grouped_gemm_ragged_k with each expert's token range cut into `splits`
 * slices on its 128-row grid, for launches with fewer output tiles than CUs
 * (one group, as for a shared expert, or few small experts): the slices'
 * fp32 partial products go to `workspace` ([splits][E][M][N] fp32, 16-byte
 * aligned, fm_grouped_gemm_ragged_k_split_workspace_bytes() bytes), and a
 * second kernel sums them in slice order (the result does not depend on
 * scheduling) into out / out2 as above.  Same reference counterpart as
 * fm_grouped_gemm_ragged_k; splits in [1, 16], 1 = the unsplit launch
 * (workspace unused); the fp32-scale blockwise kind takes splits = 1 only. */
int64_t fm_grouped_gemm_ragged_k_split_workspace_bytes(int E, int64_t M, int64_t N, int splits);
int fm_grouped_gemm_ragged_k_split(int kind, const FmGemmOperand* a_t, const FmGemmOperand* b_t,
                                   const int32_t* offsets, int E, int64_t M, int64_t N,
                                   const int32_t* expert_mask, int mask_want, void* out, int64_t out_gs,
                                   void* out2, int64_t out2_gs, int64_t split_rows, int out_dtype,
                                   int64_t ld_out, int splits, void* workspace, int64_t workspace_bytes,
                                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FM_HIP_H_ */
