// Single-track attention with pair bias (AttentionPairBias, v2) for gfx950.
//
// Replaces AttentionPairBias.forward (tt_bio/boltz2.py:343-367) as used by
// PairformerLayer (tt_bio/reference.py:906-911) and the ttnn AttentionPairBias
// non-atom branch (tt_bio/tenstorrent.py:738-787, 838-853).
//
//   apb_zbias_kernel  bias[b][h][i][j] = LN(z[b,i,j]) . W_z[h]  (MFMA, one pass over z)
//   apb_attn_kernel   one wave per (b, query i, head): fp32 logits
//                     q.k/sqrt(d) + bias - 1e6*(1-mask_k), softmax, o = P v,
//                     o * sigmoid(g) written for the output projection.
//   q/k/v/g and the output projection use linear_rows_kernel (transition.hip).
#include "pf_common.h"
#include "pf_internal.h"

namespace {

constexpr int C = 128, LDSW = 136;

// One wave = 32 pairs; W_z [H][128] (H <= 32) zero-padded to 32 rows in LDS.
__global__ __launch_bounds__(256) void apb_zbias_kernel(
    const float* __restrict__ z, const float* __restrict__ lnw, const float* __restrict__ lnb,
    const op_t* __restrict__ wz, float* __restrict__ bias, int B, int N, int H, float eps) {
  __shared__ __attribute__((aligned(16))) op_t sW[32 * LDSW];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, h = lane >> 5, m = lane & 31;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int c = tid + 256 * q;
    const int row = c >> 4;
    st_x8(&sW[row * LDSW + (c & 15) * 8], row < H ? ld_x8(wz + row * C + (c & 15) * 8) : zero_x8());
  }
  __syncthreads();
  const long NN = (long)N * N;
  const long pos0 = ((long)blockIdx.x * 4 + wid) * 32;
  if (pos0 >= (long)B * NN) return;
  const int b = (int)(pos0 / NN);
  const long t0 = pos0 - (long)b * NN;   // i*N + j of position 0
  float x[64];
  opx8 xf[8];
  load_row128_frag(z + (pos0 + m) * C, h, x);
  ln128_to_frag(x, h, lnw, lnb, eps, xf);
  f32x16 acc = zero16();
#pragma unroll
  for (int s = 0; s < 8; ++s) acc = mfma32(ld_x8(&sW[m * LDSW + 16 * s + 8 * h]), xf[s], acc);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int hd = acc_row(r, h);
    if (hd < H) bias[((long)b * H + hd) * NN + t0 + m] = acc[r];
  }
}

// One wave per (b, i, head).  Logits staged in LDS (N <= 4096).  DH = head dim.
template <int DH>
__global__ __launch_bounds__(256) void apb_attn_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ g, const float* __restrict__ bias, const float* __restrict__ mask,
    float* __restrict__ og, int B, int N, int n_valid, int c_s, int H, float inf) {
  extern __shared__ float slog[];   // [4][N]
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const long task = (long)blockIdx.x * 4 + wid;
  if (task >= (long)B * N * H) return;
  const int hd = (int)(task % H);
  const long bi = task / H;          // b*N + i
  const int b = (int)(bi / N), i = (int)(bi - (long)b * N);
  constexpr int dh = DH;
  float* lg = slog + wid * N;
  const float scale = rsqrtf((float)dh);
  const float* qp = q + bi * c_s + hd * dh;
  const float* bp = bias + (((long)b * H + hd) * N + i) * N;
  float mx = -INFINITY;
  for (int j = lane; j < n_valid; j += 64) {   // keys >= n_valid are boundary padding
    const float* kp = k + ((long)b * N + j) * c_s + hd * dh;
    float dot = 0.f;
#pragma unroll
    for (int d = 0; d < dh; ++d) dot += qp[d] * kp[d];
    float l = dot * scale + bp[j];
    if (mask) l += (1.f - mask[(long)b * N + j]) * -inf;
    lg[j] = l;
    mx = fmaxf(mx, l);
  }
  mx = wave_max(mx);
  float sum = 0.f;
  float acc[DH];
#pragma unroll
  for (int d = 0; d < dh; ++d) acc[d] = 0.f;
  for (int j = lane; j < n_valid; j += 64) {
    const float p = __expf(lg[j] - mx);
    sum += p;
    const float* vp = v + ((long)b * N + j) * c_s + hd * dh;
#pragma unroll
    for (int d = 0; d < dh; ++d) acc[d] += p * vp[d];
  }
  const float inv = 1.f / wave_sum(sum);
#pragma unroll
  for (int d = 0; d < dh; ++d) {
    const float od = wave_sum(acc[d]) * inv;
    if (lane == 0) {
      const long idx = bi * c_s + hd * dh + d;
      og[idx] = od * sigmoidf_fast(g[idx]);
    }
  }
}

}  // namespace

// linear_rows (transition.hip)
extern "C" int pf_linear_fwd(const float* x, const void* W, const float* bias, const float* resid, float* out,
                             long rows, int K, int Nout, void* stream);

extern "C" size_t pf_apb_workspace_size(int B, int N, int c_s, int H) {
  if (B <= 0 || N <= 0 || c_s <= 0 || H <= 0) return 0;
  const size_t rows = (size_t)B * N;
  return (5 * rows * c_s + (size_t)B * H * N * N) * sizeof(float);
}

extern "C" int pf_apb_fwd(const pf_apb_args* a) {
  if (!a) return pf_fail(PF_E_INVALID, "pf_apb_fwd: null args");
  if (a->B <= 0 || a->N <= 0 || a->C != C || a->H <= 0 || a->H > 32 || a->c_s % a->H ||
      (a->c_s / a->H != 24 && a->c_s / a->H != 32) || a->c_s % 32 || a->N > 4096 || (a->N % 32))
    return pf_fail(PF_E_INVALID, "pf_apb_fwd: unsupported shape B=%d N=%d c_s=%d C=%d H=%d", a->B, a->N, a->c_s,
                   a->C, a->H);
  if (!a->s || !a->k_in || !a->z || !a->out || !a->w_q || !a->b_q || !a->w_k || !a->w_v || !a->w_g ||
      !a->w_o || !a->zln_w || !a->zln_b || !a->w_z || !a->workspace)
    return pf_fail(PF_E_INVALID, "pf_apb_fwd: null pointer argument");
  if (a->n_valid < 0 || a->n_valid > a->N)
    return pf_fail(PF_E_INVALID, "pf_apb_fwd: n_valid %d outside [0, N=%d]", a->n_valid, a->N);
  const int n_valid = a->n_valid ? a->n_valid : a->N;
  const size_t need = pf_apb_workspace_size(a->B, a->N, a->c_s, a->H);
  if (a->workspace_bytes < need)
    return pf_fail(PF_E_INVALID, "pf_apb_fwd: workspace too small (%zu < %zu bytes)", a->workspace_bytes, need);
  hipStream_t st = (hipStream_t)a->stream;
  const long rows = (long)a->B * a->N;
  const int cs = a->c_s;
  float* q = (float*)a->workspace;
  float* k = q + rows * cs;
  float* v = k + rows * cs;
  float* g = v + rows * cs;
  float* og = g + rows * cs;
  float* bias = og + rows * cs;
  int rc;
  if ((rc = pf_linear_fwd(a->s, a->w_q, a->b_q, nullptr, q, rows, cs, cs, a->stream))) return rc;
  if ((rc = pf_linear_fwd(a->k_in, a->w_k, nullptr, nullptr, k, rows, cs, cs, a->stream))) return rc;
  if ((rc = pf_linear_fwd(a->k_in, a->w_v, nullptr, nullptr, v, rows, cs, cs, a->stream))) return rc;
  if ((rc = pf_linear_fwd(a->s, a->w_g, nullptr, nullptr, g, rows, cs, cs, a->stream))) return rc;
  const long pairs = (long)a->B * a->N * a->N;
  apb_zbias_kernel<<<(unsigned)((pairs / 32 + 3) / 4), 256, 0, st>>>(a->z, a->zln_w, a->zln_b, (const op_t*)a->w_z,
                                                                    bias, a->B, a->N, a->H, a->eps);
  PF_CHECK_LAUNCH("apb_zbias_kernel");
  const long tasks = rows * a->H;
  const unsigned grid = (unsigned)((tasks + 3) / 4);
  const size_t lds = 4 * a->N * sizeof(float);
  if (cs / a->H == 24)
    apb_attn_kernel<24><<<grid, 256, lds, st>>>(q, k, v, g, bias, a->mask, og, a->B, a->N, n_valid, cs, a->H, 1e6f);
  else
    apb_attn_kernel<32><<<grid, 256, lds, st>>>(q, k, v, g, bias, a->mask, og, a->B, a->N, n_valid, cs, a->H, 1e6f);
  PF_CHECK_LAUNCH("apb_attn_kernel");
  return pf_linear_fwd(og, a->w_o, nullptr, a->accumulate ? a->out : nullptr, a->out, rows, cs, cs, a->stream);
}
