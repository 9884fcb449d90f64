/*
 * pairformer_hip.h -- C ABI of libpairformer_hip.so, the MI355X (gfx950) kernels for
 * the Boltz-2 Pairformer pair-representation hot path.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers (HIP global memory) unless stated otherwise.
 *   - Dense row-major layouts.  Pair tensors are [B][N][N][C] fp32; masks are fp32 0/1.
 *   - Matrix weights are in the library's MFMA operand type (raw 16-bit patterns):
 *     IEEE fp16 in libpairformer_hip.so, bf16 in libpairformer_hip_bf16.so
 *     (pf_operand_dtype() says which), nn.Linear layout [out][in].  LayerNorm
 *     weights/biases and linear biases are fp32.  Accumulation is fp32 everywhere.
 *     Weight names in the comments are the reference state-dict keys
 *     (tt_bio/reference.py, tt_bio/boltz2.py); "bf16"/"op" below means the operand type.
 *   - `stream` is a hipStream_t (NULL = default stream).  Calls only enqueue work;
 *     they do not synchronize and do not allocate device memory.  Scratch memory is
 *     passed in as `workspace` (size from the matching *_workspace_size()).
 *   - Return 0 on success or a negative PF_E_* code; pf_last_error() then returns a
 *     thread-local message.  Nothing is launched when an argument is rejected.
 *   - N (tokens) must be a positive multiple of 64: the Python boundary pads to 64
 *     like the reference does (tt_bio/tenstorrent.py:41, 2235-2246).
 *   - `accumulate`: 0 -> out = update, 1 -> out += update.  out may alias the input
 *     pair tensor (in-place residual, `z = z + op(z)` in tt_bio/reference.py:877-903).
 *   - `n_valid` (attention entry points): tokens >= n_valid are boundary padding and
 *     are excluded from every softmax (weight exactly 0), so a row whose valid keys are
 *     all masked still averages over the n_valid real keys as the unpadded reference
 *     does.  0 means N (no padding).
 */
#ifndef PAIRFORMER_HIP_H
#define PAIRFORMER_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PF_ABI_VERSION 3

enum {
  PF_OK = 0,
  PF_E_INVALID = -1, /* bad shape / null pointer / unsupported configuration */
  PF_E_OOM = -2,     /* reserved: message contains "out of memory" */
  PF_E_LAUNCH = -3   /* a kernel launch failed (message names the kernel) */
};

/* ABI version of the loaded library (PF_ABI_VERSION at build time). */
int pf_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* pf_last_error(void);

/* MFMA operand type of this build: 0 = IEEE fp16, 1 = bf16. */
int pf_operand_dtype(void);

/* ------------------------------------------------------------------------------
 * Triangle multiplication, outgoing (direction 0) and incoming (direction 1).
 * Replaces TriangleMultiplicationOutgoing/Incoming.forward
 * (tt_bio/reference.py:455-472, 544-561), the ttnn TriangleMultiplication.__call__
 * (tt_bio/tenstorrent.py:409-503) and the fused-op contract
 * kernel_triangular_mult(x, direction, mask, norm_in_weight, norm_in_bias,
 * p_in_weight, g_in_weight, norm_out_weight, norm_out_bias, p_out_weight,
 * g_out_weight, eps) (tt_bio/boltz2.py:820-848).
 *   update = p_out(LN_out(x)) * sigmoid(g_out(LN_in(z))),
 *   x[i,j] = sum_k a[i,k]*b[j,k] (outgoing) or sum_k a[k,i]*b[k,j] (incoming),
 *   a|b = p_in(LN_in z) * sigmoid(g_in(LN_in z)) * pair_mask.
 * -------------------------------------------------------------------------- */
typedef struct pf_trimul_args {
  int B, N, C;            /* C = c_z = 128 */
  int hidden;             /* must equal C (Boltz-2: p_in is [2*C, C]) */
  int direction;          /* 0 outgoing, 1 incoming */
  int accumulate;
  float eps;              /* LayerNorm eps (1e-5) */
  const float* z_in;      /* [B][N][N][C] */
  float* out;             /* [B][N][N][C], may alias z_in */
  const float* pair_mask; /* [B][N][N] or NULL (all ones) */
  const float* norm_in_w; const float* norm_in_b;    /* norm_in.{weight,bias} [C] */
  const void* p_in_w;     /* p_in.weight  bf16 [2C][C] */
  const void* g_in_w;     /* g_in.weight  bf16 [2C][C] */
  const float* norm_out_w; const float* norm_out_b;  /* norm_out.{weight,bias} [C] */
  const void* p_out_w;    /* p_out.weight bf16 [C][C] */
  const void* g_out_w;    /* g_out.weight bf16 [C][C] */
  void* workspace; size_t workspace_bytes;
  void* stream;
  /* Optional (NULL = unused; C = 128 only): the residual p_out - p_out16 of p_out.weight,
   * rounded to the operand type.  The output projection then runs on p_out16 + residual (two
   * MFMAs per fragment), with weights good to ~2^-22 of their size (see pf_triatt_args). */
  const void* p_out_lo;
  /* Optional (NULL = unused; C = 128 only): in_offsets fp32 [5C] = p_in.weight . beta [2C],
   * g_in.weight . beta [2C], g_out.weight . beta [C] in fp32 from the unrounded weights (beta =
   * norm_in.bias); the kernels then add these instead of the 16-bit weights' W16 . beta.  With
   * also the residuals p_in_lo, g_in_lo, g_out_lo (W - W16 in the operand type) and B == 1,
   * the mean correction: each of those rows' offsets also gets W_lo . (norm_in.weight * mu),
   * mu = the mean over positions of the normalized z (estimated from up to 32768 sampled
   * positions): the part of a 16-bit weight's rounding error that every position shares. */
  const float* in_offsets;
  const void* p_in_lo; const void* g_in_lo; const void* g_out_lo;
} pf_trimul_args;

size_t pf_trimul_workspace_size(int B, int N, int C);
int pf_trimul_fwd(const pf_trimul_args* args);

/* The contraction alone: X[p][i][j] = sum_k A[p][i][k] * Bm[p][j][k] for `planes`
 * independent N x N operand-type planes.  x_fp32 = 1: X is fp32; x_fp32 = 0: X is the
 * operand type scaled by 2^-8 (pf_trimul_fwd itself scales its X planes by a per-call power of
 * two chosen from the largest |a|, |b| it wrote).  The batched
 * matmul inside TriangleMultiplication (tt_bio/tenstorrent.py:453-460; einsum at
 * tt_bio/reference.py:467, 556). */
int pf_trimul_contract(const void* A, const void* Bm, void* X, int x_fp32, int planes, int N, void* stream);

/* ------------------------------------------------------------------------------
 * Triangle attention, starting node (ending = 0) and ending node (ending = 1).
 * Replaces TriangleAttention.forward (tt_bio/reference.py:294-365, with
 * Attention.forward 138-194 and _attention tt_bio/boltz2.py:790-810) and the ttnn
 * TriangleAttention.__call__ (tt_bio/tenstorrent.py:541-650).
 *   x = LN(z) (z transposed for the ending node); per row i, head h, query j:
 *   logits_k = (q_ij/sqrt(d)).k_ik + 1e9*(pair_mask_ik - 1) + (x_jk . w_b[h]);
 *   softmax over k (fp32, online); o = sum_k p_k v_ik; update = linear_o(o * sigmoid(g)).
 * -------------------------------------------------------------------------- */
typedef struct pf_triatt_args {
  int B, N, C;            /* C = 128 */
  int H, D;               /* heads = 4, head dim = 32 (H*D == C) */
  int ending;             /* 0 starting node, 1 ending node */
  int accumulate;
  int n_valid;            /* keys >= n_valid excluded (boundary padding); 0 = N */
  float eps;
  const float* z_in;      /* [B][N][N][C] */
  float* out;             /* may alias z_in */
  const float* pair_mask; /* [B][N][N] or NULL */
  const float* ln_w; const float* ln_b;   /* layer_norm.{weight,bias} [C] */
  const void* w_bias;     /* linear.weight      bf16 [H][C] */
  const void* w_q; const void* w_k; const void* w_v; const void* w_g;  /* mha.linear_{q,k,v,g}.weight bf16 [H*D][C] */
  const void* w_o;        /* mha.linear_o.weight bf16 [C][H*D] */
  void* workspace; size_t workspace_bytes;
  void* stream;
  /* Optional (NULL = unused; C = 128 only): the residuals W - W16 of linear_g and linear_o,
   * rounded to the operand type.  With both given, the gate and the output projection run on
   * W16 + residual (two MFMAs per fragment), i.e. with weights good to ~2^-22 of their size:
   * the 2^-12 rounding of 16-bit weights is the same at every position, and it is what makes
   * a deep stack drift from the fp32 reference. */
  const void* w_g_lo; const void* w_o_lo;
  /* Optional (NULL = unused; C = 128 only): in_offsets fp32 [3C + H] = linear_q / _k / _v
   * .weight . beta and linear.weight . beta in fp32 from the unrounded weights (beta =
   * layer_norm.bias), used instead of the 16-bit weights' W16 . beta; with also the residuals
   * of the kernel's gamma-folded weights, w_*_lo = W diag(gamma) - op(op(W) diag(gamma)) in the
   * operand type (op = rounding to it; [H*D][C] for q, k, v, [H][C] for the bias), and B == 1,
   * the mean correction of pf_trimul_args for those rows. */
  const float* in_offsets;
  const void* w_q_lo; const void* w_k_lo; const void* w_v_lo; const void* w_bias_lo;
} pf_triatt_args;

size_t pf_triatt_workspace_size(int B, int N, int C, int H, int D);
int pf_triatt_fwd(const pf_triatt_args* args);

/* The flash-attention kernel of pf_triatt_fwd alone (the softmax(q.k + bias + mask).v core
 * of tt_bio/reference.py:176-190 / tt_bio/boltz2.py:790-810 inside TriangleAttention), run on
 * the q, k, v, bias and mask that the last pf_triatt_fwd call with the same B and N left in
 * `workspace`; its output goes to the same workspace.  Exported for measurement of the
 * dominant kernel on its real operands. */
int pf_triatt_attend_workspace(void* workspace, size_t workspace_bytes, int B, int N, int n_valid, void* stream);

/* Attention core with the signature of the fused-op contract
 * kernel_triangular_attn(q, k, v, tri_bias, mask, scale) (tt_bio/boltz2.py:815-817)
 * and the semantics of the use_kernels=False path it stands in for
 * (tt_bio/reference.py:176-190, tt_bio/boltz2.py:790-810):
 *   o[b,i,h,j,:] = sum_k softmax_k(scale*q.k + 1e9*(mask[b,i,k]-1) + bias[b,h,j,k]) v[b,i,h,k,:]
 * q, k, v: fp32 [B][I][H][J][D] (I = J = N); bias fp32 [B][H][N][N]; mask fp32 [B][I][N]
 * or NULL; o fp32 [B][I][H][J][D].  D must be 32; keys >= n_valid are padding (0 = N). */
size_t pf_tri_attention_workspace_size(int B, int N, int H, int D);
int pf_tri_attention(const float* q, const float* k, const float* v, const float* bias,
                     const float* mask, float scale, float* o, int B, int N, int H, int D,
                     int n_valid, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------
 * Transition (SwiGLU MLP): update = fc3(silu(fc1(LN(x))) * fc2(LN(x))), no biases.
 * Replaces Transition.forward (tt_bio/boltz2.py:1227-1258) and the ttnn Transition
 * (tt_bio/tenstorrent.py:856-946).  rows = B*N*N for the pair track (C = 128,
 * hidden = 512: one fused kernel, hidden never leaves the CU) or B*N for the single
 * track (C = 384, hidden = 1536: LN + two GEMMs, hidden in workspace).  The C = 128
 * workspace (256.5 KB whatever rows) is used only by fc3_mean_fix.
 * -------------------------------------------------------------------------- */
typedef struct pf_transition_args {
  long rows; int C; int hidden;
  int accumulate;
  float eps;
  const float* x_in;      /* [rows][C] */
  float* out;             /* [rows][C], may alias x_in */
  const float* norm_w; const float* norm_b;   /* norm.{weight,bias} [C] */
  const void* fc1_w; const void* fc2_w;       /* bf16 [hidden][C] */
  const void* fc3_w;                          /* bf16 [C][hidden] */
  void* workspace; size_t workspace_bytes;
  void* stream;
  /* Optional (NULL = unused; C = 128 only): the residual fc3 - fc3_16 of fc3.weight in the
   * operand type; the output projection then runs on fc3_16 + residual (see pf_triatt_args). */
  const void* fc3_lo;
  /* With fc3_lo: 0 = multiply by fc3_16 + residual at every position; 1 = multiply by fc3_16
   * and add residual . mean(h), h = silu(fc1 LN(x)) * fc2 LN(x) averaged over up to 256 sampled
   * tiles of 32 consecutive rows (a pass over those rows before the main one): the part of the
   * residual's error that every position shares, at a fraction of the cost.  The sample is
   * drawn from all rows (with B > 1 the batch elements' means are pooled; the Python module
   * uses it for one batch element).  Needs the workspace (pf_transition_workspace_size;
   * C = 128) and hidden a multiple of 64, <= 512. */
  int fc3_mean_fix;
} pf_transition_args;

size_t pf_transition_workspace_size(long rows, int C, int hidden);
int pf_transition_fwd(const pf_transition_args* args);

/* ------------------------------------------------------------------------------
 * Single-track attention with pair bias (AttentionPairBias, v2, compute_pair_bias).
 * Replaces AttentionPairBias.forward (tt_bio/boltz2.py:343-367) as called from
 * PairformerLayer.forward (tt_bio/reference.py:906-911) and the ttnn
 * AttentionPairBias (tt_bio/tenstorrent.py:738-853, non-atom branch):
 *   q = proj_q(s) + b_q, k = proj_k(k_in), v = proj_v(k_in),
 *   bias = proj_z.1(LN_{proj_z.0}(z)) [B,H,N,N],
 *   logits = q.k/sqrt(d) + bias - 1e6*(1 - mask_k), softmax, o = P v,
 *   update = proj_o(sigmoid(proj_g(s)) * o).
 * s, k_in fp32 [B][N][c_s]; z fp32 [B][N][N][C]; mask fp32 [B][N] or NULL.
 * -------------------------------------------------------------------------- */
typedef struct pf_apb_args {
  int B, N, c_s, C, H;    /* c_s = 384, C = 128, H = 16 (head dim c_s/H) */
  int accumulate;
  int n_valid;            /* keys >= n_valid excluded (boundary padding); 0 = N */
  float eps;              /* eps of the proj_z LayerNorm */
  const float* s;         /* query input (pre_norm_s(s) in the Pairformer) */
  const float* k_in;      /* key/value input */
  const float* z;         /* pair tensor */
  const float* mask;      /* [B][N] or NULL */
  float* out;             /* [B][N][c_s], may alias neither s nor k_in when accumulate=0 */
  const void* w_q; const float* b_q;          /* proj_q.{weight bf16 [c_s][c_s], bias fp32} */
  const void* w_k; const void* w_v; const void* w_g; const void* w_o;  /* bf16 [c_s][c_s] */
  const float* zln_w; const float* zln_b;     /* proj_z.0.{weight,bias} [C] */
  const void* w_z;                            /* proj_z.1.weight bf16 [H][C] */
  void* workspace; size_t workspace_bytes;
  void* stream;
} pf_apb_args;

size_t pf_apb_workspace_size(int B, int N, int c_s, int H);
int pf_apb_fwd(const pf_apb_args* args);

/* pf_apb_fwd in two halves, for callers that overlap the single track with the next
 * layer's pair operations on a second stream: pf_apb_pair_bias computes the z-dependent
 * part (bias = proj_z.1(LN(z)), tt_bio/boltz2.py:353-356) into the workspace, and
 * pf_apb_attend runs the rest (boltz2.py:343-352, 357-367) with that bias, on its own
 * stream (args->stream of each call).  Same arguments for both (pf_apb_pair_bias reads
 * only the shape, z, zln_w, zln_b, w_z, eps, workspace and stream); the caller orders
 * pf_apb_attend after pf_apb_pair_bias and the next pf_apb_pair_bias after the previous
 * pf_apb_attend on one workspace.  pf_apb_fwd(a) == pf_apb_pair_bias(a); pf_apb_attend(a). */
int pf_apb_pair_bias(const pf_apb_args* args);
int pf_apb_attend(const pf_apb_args* args);

/* pf_apb_fwd for callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops that forbid hipMalloc).  No counterpart in the reference.  Same arguments and
 * result as pf_apb_fwd, except that args->workspace / workspace_bytes are ignored: the scratch
 * is a static device array of PF_APB_NOALLOC_SCRATCH_BYTES per GPU, which holds
 * pf_apb_workspace_size(B, N, c_s, H) up to that size (e.g. B = 1, N = 512, c_s = 384,
 * H = 16: 20.7 MiB); larger shapes are rejected with PF_E_INVALID.  Allocates nothing; the
 * array lives until the process ends.  Every call on one GPU shares that GPU's scratch, so
 * calls that overlap on one GPU (other streams or threads) race: serialize them.  The scratch
 * needs no clearing (each call writes every byte it reads). */
#define PF_APB_NOALLOC_SCRATCH_BYTES (24u << 20)
int pf_apb_fwd_noalloc(const pf_apb_args* args);

/* The pair transition (pf_transition_fwd, C = 128 only) with pf_apb_pair_bias of its
 * result fused into the same kernel: after writing out = [x_in +] Transition(x_in) for a
 * pair, the kernel also writes that pair's single-track bias log2(e)*proj_z(LN(out)) into
 * apb's workspace, as pf_apb_pair_bias(apb) on `out` would (tt_bio/boltz2.py:353-356), so
 * the layer's last pair operation and the single track's only z read are one pass.
 * apb: shape, zln_w, zln_b, w_z, eps, workspace (the other fields are not read; apb->z is
 * ignored: the bias is computed from t->out).  t->rows must equal apb->B * apb->N^2. */
int pf_transition_pair_bias_fwd(const pf_transition_args* t, const pf_apb_args* apb);

/* ------------------------------------------------------------------------------
 * Fast mode (block fp8).  Replaces the --fast path of the ttnn TriangleMultiplication
 * and Transition (tt_bio/tenstorrent.py:60-61, 178-181, 389-407, 431-503, 879-906),
 * which the reference selects with set_fast_mode() before building the modules
 * (tt_bio/worker.py:151-153) and which has no CPU counterpart (tt_bio/main.py:1648-1649).
 * Format: OCP MXFP8 -- e4m3 elements (round to nearest even, saturating at +-448) with
 * one E8M0 scale byte per 32 consecutive elements along the contraction axis:
 * the smallest power of two X with amax / X <= 448 (OCP MX's floor(log2(amax)) - 8,
 * one higher when amax's significand exceeds 1.75, so no element saturates);
 * fp32 accumulation.  Matrices are passed pre-quantized
 * (pf_quantize_mx8): q = e4m3 bytes [rows][K], s = scale bytes [rows][K/32].
 * -------------------------------------------------------------------------- */

/* Quantize x fp32 [rows][K] (K % 32 == 0) along K: q bytes [rows][K], scales [rows][K/32].
 * perm = 0 keeps the element order; perm = 1 stores each 32-block in accumulator order
 * (destination 16h + 4j + e <- source 4h + 8j + e), the order pf_transition_mx8_fwd
 * expects for fc3.weight.  Asynchronous on `stream`. */
int pf_quantize_mx8(const float* x, long rows, int K, int perm, void* q, void* scales, void* stream);

/* Triangle multiplication with MXFP8 projections and contraction operands (same
 * semantics and argument meaning as pf_trimul_fwd; N must be a multiple of 128).
 * Quantized: LN_in(z) and p_in/g_in (K = C); a and b along the contraction index;
 * LN_out(x) and p_out; LN_in(z) and g_out. */
typedef struct pf_trimul_mx8_args {
  int B, N, C, hidden, direction, accumulate;
  float eps;
  const float* z_in; float* out; const float* pair_mask;
  const float* norm_in_w; const float* norm_in_b;
  const void* p_in_q; const void* p_in_s;     /* p_in.weight  [2C][C] e4m3, [2C][C/32] E8M0 */
  const void* g_in_q; const void* g_in_s;     /* g_in.weight */
  const float* norm_out_w; const float* norm_out_b;
  const void* p_out_q; const void* p_out_s;   /* p_out.weight [C][C], [C][C/32] */
  const void* g_out_q; const void* g_out_s;   /* g_out.weight */
  void* workspace; size_t workspace_bytes;
  void* stream;
} pf_trimul_mx8_args;

size_t pf_trimul_mx8_workspace_size(int B, int N, int C);
int pf_trimul_mx8_fwd(const pf_trimul_mx8_args* args);

/* The MXFP8 contraction alone (tests): X fp32 [planes][N][N] = A . B^T per plane, A/B e4m3
 * [planes][N][N] with scales [planes][N][N/32] along the last axis; N % 128 == 0. */
int pf_trimul_mx8_contract(const void* A8, const void* B8, const void* SA, const void* SB, float* X,
                           int planes, int N, void* stream);

/* Pair transition with MXFP8 GEMMs (C = 128, hidden % 64 == 0): LN(x) and fc1/fc2 (K = C),
 * silu(fc1)*fc2 and fc3 (K = hidden).  fc3 must be quantized with perm = 1. */
typedef struct pf_transition_mx8_args {
  long rows; int C; int hidden; int accumulate;
  float eps;
  const float* x_in; float* out;
  const float* norm_w; const float* norm_b;
  const void* fc1_q; const void* fc1_s;       /* fc1.weight [hidden][C] */
  const void* fc2_q; const void* fc2_s;       /* fc2.weight [hidden][C] */
  const void* fc3_q; const void* fc3_s;       /* fc3.weight [C][hidden], perm = 1 */
  void* stream;
} pf_transition_mx8_args;

int pf_transition_mx8_fwd(const pf_transition_mx8_args* args);

/* pf_transition_mx8_fwd with the single-track pair bias of its result fused in, as
 * pf_transition_pair_bias_fwd does for the 16-bit transition: after writing a pair of out,
 * the kernel also writes that pair's log2(e)*proj_z(LN(out)) into apb's workspace (the
 * projection in the operand type, as pf_apb_pair_bias computes it).  t->rows must equal
 * apb->B * apb->N^2 and be a multiple of 128. */
int pf_transition_mx8_pair_bias_fwd(const pf_transition_mx8_args* t, const pf_apb_args* apb);

/* Triangle attention in fast mode (same semantics and argument meaning as pf_triatt_fwd,
 * C = 128).  The block-fp8 points are those of the ttnn TriangleAttention under --fast
 * (tt_bio/tenstorrent.py:526-539 weights, 603-614 / 628-639 projections, 580-590 output):
 * linear_{q,k,v,g}.weight MXFP8 along C (pf_quantize_mx8, dequantized per call into the
 * workspace, so the LayerNorm output stays 16-bit as in the reference); q, k, v and g
 * quantize-dequantized per head (32 channels) right after their projections; the
 * o-projection's output per 32 channels before the residual.  linear.weight (the triangle
 * bias) and linear_o.weight stay 16-bit, as the reference keeps them bfloat16. */
typedef struct pf_triatt_mx8_args {
  int B, N, C;            /* C = 128 */
  int H, D;               /* heads = 4, head dim = 32 */
  int ending;
  int accumulate;
  int n_valid;
  float eps;
  const float* z_in;
  float* out;
  const float* pair_mask;
  const float* ln_w; const float* ln_b;
  const void* w_bias;                        /* linear.weight op_t [H][C] */
  const void* w_q_q; const void* w_q_s;      /* mha.linear_q.weight [H*D][C] e4m3, [H*D][C/32] E8M0 */
  const void* w_k_q; const void* w_k_s;
  const void* w_v_q; const void* w_v_s;
  const void* w_g_q; const void* w_g_s;
  const void* w_o;                           /* mha.linear_o.weight op_t [C][H*D] */
  void* workspace; size_t workspace_bytes;
  void* stream;
} pf_triatt_mx8_args;

size_t pf_triatt_mx8_workspace_size(int B, int N, int C, int H, int D);
int pf_triatt_mx8_fwd(const pf_triatt_mx8_args* args);

/* AttentionPairBias in fast mode: pf_apb_fwd / pf_apb_attend with o * sigmoid(g)
 * quantize-dequantized along c_s (32-channel blocks) before the output projection, the
 * reference's multiply(..., dtype=_dtype()) (tt_bio/tenstorrent.py:844-846).  c_s % 32 == 0. */
int pf_apb_fwd_mx8(const pf_apb_args* args);
int pf_apb_attend_mx8(const pf_apb_args* args);

/* ------------------------------------------------------------------------------
 * MSA module (widening beyond the Pairformer: tt_bio/reference.py:1150-1398, the ttnn
 * MSA / MSALayer in tt_bio/tenstorrent.py:1723-1855).
 * -------------------------------------------------------------------------- */
/* Outer product mean (OuterProductMean.forward, tt_bio/reference.py:596-664; ttnn
 * tt_bio/tenstorrent.py:1632-1720, which divides by the sequence count instead of the
 * per-pair mask count -- this follows the CPU reference):
 *   z[b,i,j,:] (+)= W_o vec_{c,d}(sum_s a[s,i,c] b[s,j,d]) / max(1, sum_s mask[s,i] mask[s,j]) + b_o,
 *   a = W_a LN(m) * mask, b = W_b LN(m) * mask.
 * m fp32 [B][S][N][c_m], msa_mask fp32 [B][S][N] or NULL (all ones), z fp32 [B][N][N][C]
 * updated in place (accumulate = 1) or overwritten.  c_m = 64, c_hidden = 32, C = 128,
 * N a multiple of 32, any S. */
typedef struct pf_opm_args {
  int B, S, N, c_m, c_hidden, C;
  int accumulate;
  float eps;
  const float* m; const float* msa_mask; float* z;
  const float* norm_w; const float* norm_b;   /* norm.{weight,bias} [c_m] */
  const void* w_a; const void* w_b;           /* proj_{a,b}.weight [c_hidden][c_m] */
  const void* w_o; const float* b_o;          /* proj_o.weight [C][c_hidden^2], bias [C] fp32 */
  void* workspace; size_t workspace_bytes;
  void* stream;
} pf_opm_args;

size_t pf_opm_workspace_size(int B, int S, int N);
int pf_opm_fwd(const pf_opm_args* args);

/* Pair weighted averaging (PairWeightedAveraging.forward, tt_bio/reference.py:715-790;
 * ttnn tt_bio/tenstorrent.py:1757-1796 callers):
 *   w[h,i,j] = softmax_j(LN_z(z[i,j]) . W_z[h] - 1e6 (1 - pair_mask[i,j])),
 *   o[s,i,h,:] = sigmoid(W_g LN_m(m[s,i]))_h * sum_j w[h,i,j] (W_m LN_m(m[s,j]))_h,
 *   out[s,i,:] = (accumulate ? m[s,i,:] : 0) + W_o o[s,i,:]   (out may alias m).
 * m fp32 [B][S][N][c_m], z fp32 [B][N][N][C], pair_mask fp32 [B][N][N] or NULL.
 * c_m = 64, C = 128, H = 8 heads of c_h = 32, N a multiple of 64, any S. */
typedef struct pf_pwa_args {
  int B, S, N, c_m, C, H, c_h;
  int accumulate;
  float eps;
  const float* m; float* out; const float* z; const float* pair_mask;
  const float* norm_m_w; const float* norm_m_b;   /* norm_m.{weight,bias} [c_m] */
  const float* norm_z_w; const float* norm_z_b;   /* norm_z.{weight,bias} [C] */
  const void* w_m; const void* w_g;               /* proj_{m,g}.weight [H*c_h][c_m] */
  const void* w_z;                                /* proj_z.weight [H][C] */
  const void* w_o;                                /* proj_o.weight [c_m][H*c_h] */
  void* workspace; size_t workspace_bytes;
  void* stream;
} pf_pwa_args;

size_t pf_pwa_workspace_size(int B, int S, int N);
int pf_pwa_fwd(const pf_pwa_args* args);

/* MSA input embedding (MSAModule.forward, tt_bio/reference.py:1253-1276, with
 * use_paired_feature): m[b,s,i,:] = msa_proj([one_hot(msa), has_deletion, deletion_value,
 * is_paired]) + s_emb[b,i,:], as a column gather.  msa int32 [B][S][N] token ids
 * (clamped to [0, n_tok)); the three features fp32 [B][S][N] or NULL (zero); s_emb fp32
 * [B][N][c_m] (= s_proj(emb), e.g. by pf_linear_fwd); w_t fp32 [n_tok + 3][c_m] = msa_proj.weight
 * transposed; m fp32 [B][S][N][c_m].  c_m = 64. */
int pf_msa_embed(const int* msa, const float* has_deletion, const float* deletion_value, const float* msa_paired,
                 const float* s_emb, const float* w_t, float* m, int B, int S, int N, int c_m, int n_tok,
                 void* stream);

/* Batched NT product X[p][i][j] = scale * sum_k A[p][i][k] * B[p][j][k] on the MFMA
 * contraction kernel: A [planes][M][K], B [planes][Nc][K] in the operand type, X
 * [planes][M][Nc] fp32 (x_fp32 = 1) or operand type; M, Nc multiples of 32, K a multiple of
 * 64.  No single reference counterpart: it is the building block of the MSA module's
 * einsums "bsic,bsjd->bijcd" (tt_bio/reference.py:656) and "bhij,bhsjd->bhsid" (:786),
 * exported for tests and measurement.  Asynchronous on `stream`. */
int pf_batched_nt_gemm(const void* A, const void* B, void* X, int x_fp32, int planes, int M, int Nc, int K,
                       float scale, void* stream);

/* ------------------------------------------------------------------------------
 * Row primitives (tt_bio/boltz2.py:638-768): LayerNorm and Linear over rows.
 * -------------------------------------------------------------------------- */
/* out[r,:] = LN(x[r,:]) * w + b, fp32, any C <= 4096.  (nn.LayerNorm, eps) */
int pf_layernorm_fwd(const float* x, const float* w, const float* b, float* out, long rows,
                     int C, float eps, void* stream);

/* out[r,n] = (resid ? resid[r,n] : 0) + sum_k x[r,k] * W[n,k] + (bias ? bias[n] : 0).
 * x fp32 [rows][K], W bf16 [Nout][K], K a multiple of 16, Nout a multiple of 32.
 * resid may alias out.  (nn.Linear) */
int pf_linear_fwd(const float* x, const void* W, const float* bias, const float* resid,
                  float* out, long rows, int K, int Nout, void* stream);

/* Pair-track recycling step of the trunk loop (tt_bio/boltz2.py:5213-5214):
 *   out[p,:] = base[p,:] + W . LN(x[p,:])   for every pair p, C = 128.
 * (z = z_init + z_recycle(z_norm(z))); out may alias x but not base unless equal.
 * W_lo (optional, NULL = unused): the residual W - W16 in the operand type; with it the product
 * takes both the weight and the normalized activation as 16-bit hi + lo pairs (three MFMAs per
 * fragment), i.e. it is computed to ~fp32 accuracy.  At a pass's start z is zero, LN(z) is the
 * same beta at every pair, and a 16-bit rounding of W or beta would shift every pair alike. */
int pf_pair_ln_linear_fwd(const float* x, const float* base, const float* ln_w, const float* ln_b,
                          const void* W, const void* W_lo, float* out, long rows, int C, float eps, void* stream);

/* ------------------------------------------------------------------------------
 * Diffusion conditioning, pair side (run once per trunk output; fixed for every
 * sampling step).  z, rel_pos, out: fp32 [rows][128] (rows = B*N*N); LN params fp32.
 * -------------------------------------------------------------------------- */
/* PairwiseConditioning input projection (tt_bio/boltz2.py:1330-1333, 1349-1350):
 *   out[p,:] = W . LN(cat(z[p,:], rel_pos[p,:]))   LN over 256 channels (ln_w, ln_b [256]),
 *   W [128][256] in the operand type (LinearNoBias).  out must not alias an input. */
int pf_pair_cond_proj_fwd(const float* z, const float* rel_pos, const float* ln_w, const float* ln_b,
                          const void* W, float* out, long rows, int c_z, float eps, void* stream);

/* Token-transformer pair bias of DiffusionConditioning (tt_bio/boltz2.py:2434-2441,
 * 2472-2475; ttnn AttentionPairBias.compute_bias, tt_bio/tenstorrent.py:714-728):
 *   bias[p, l*H + h] = scale * LN_l(z[p,:]) . W[l*H + h, :]   for l < n_layers, h < n_heads
 * ln_w, ln_b [n_layers][128] (each layer's LayerNorm), W [n_layers*n_heads][128] (the layers'
 * Linear(c_z, H, bias=False) weights stacked), n_layers*n_heads a multiple of 32, <= 512.
 * layout 0: out [rows][L*H] (the reference's torch.cat(..., dim=-1)); layout 1: out
 * [L*H][rows] (one contiguous plane per layer and head). */
int pf_token_pair_bias_fwd(const float* z, const float* ln_w, const float* ln_b, const void* W, float* out,
                           long rows, int c_z, int n_layers, int n_heads, int layout, float scale, float eps,
                           void* stream);

/* Residual hand-off of the trunk loop (tt_bio/boltz2.py:5221, 5230:
 *   z = z + template_module(z, ...), z = z + msa_module(z, ...)):
 *   out[i] = a[i] + b[i], fp32, 16-byte aligned pointers; out may alias a or b. */
int pf_add_fwd(const float* a, const float* b, float* out, long n, void* stream);

/* ------------------------------------------------------------------------------
 * Measurement aids (no counterpart in the reference: they serve the benchmark's roofline
 * figures and allocate no device memory).
 * -------------------------------------------------------------------------- */
/* In-layer launch timing of the triangle-attention core: pf_attend_timing(1) clears and starts
 * the calling host thread's record, after which every ta_attn_kernel launch that thread makes
 * (pf_triatt_fwd, pf_triatt_mx8_fwd, pf_triatt_attend_workspace, pf_tri_attention) is bracketed
 * by HIP events on its stream; pf_attend_timing(0) stops recording.  pf_attend_timing_read
 * waits for the last recorded launch and returns the summed launch durations (ms) and the
 * number of launches. */
int pf_attend_timing(int enable);
int pf_attend_timing_read(double* total_ms, int* launches);

/* The same for a chosen kernel kind: PF_TIMED_ATTEND (as above), PF_TIMED_CONTRACT8 (the
 * block-fp8 contraction inside pf_trimul_mx8_fwd and pf_trimul_mx8_contract) or
 * PF_TIMED_CONTRACT (the 16-bit contraction inside pf_trimul_fwd). */
#define PF_TIMED_ATTEND 0
#define PF_TIMED_CONTRACT8 1
#define PF_TIMED_CONTRACT 2
#define PF_TIMED_KINDS 3
int pf_kernel_timing(int kind, int enable);
int pf_kernel_timing_read(int kind, double* total_ms, int* launches);

/* MFMA issue rate under load: `workgroups` workgroups of 16 waves each issue `iters` (a
 * multiple of 4) rounds of four mutually independent 32x32x16 16-bit MFMAs (pseudo-random operands in (-1, 1) that change
 * every MFMA), i.e. pf_mfma_rate_probe_waves(workgroups) * iters * 4 * 32768 FLOP; every wave
 * writes one float of `sink` (workgroups * 16 floats). */
long pf_mfma_rate_probe_waves(int workgroups);
int pf_mfma_rate_probe(int workgroups, int iters, float* sink, void* stream);
/* The same on the block-scaled fp8 MFMA (32x32x64 e4m3, unit scales): 4 * 131072 FLOP per
 * round and wave. */
int pf_mfma8_rate_probe(int workgroups, int iters, float* sink, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* PAIRFORMER_HIP_H */
