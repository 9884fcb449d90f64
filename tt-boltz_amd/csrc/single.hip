// Single-track attention with pair bias (AttentionPairBias, v2) for gfx950.
//
// Replaces AttentionPairBias.forward (tt_bio/boltz2.py:343-367) as used by
// PairformerLayer (tt_bio/reference.py:906-911) and the ttnn AttentionPairBias
// non-atom branch (tt_bio/tenstorrent.py:738-787, 838-853).
//
//   apb_zbias_kernel  bias[b][h][i][j] = log2(e) * LN(z[b,i,j]) . W_z[h]  (MFMA, one pass
//                     over z; log2 units for the exp2 softmax)
//   apb_attn_kernel   one workgroup of 8 waves per (b, head, 32 queries); wave w takes
//                     key tiles w, w + 8, ... (32 keys each): MFMA scores
//                     q.k/sqrt(d) + bias - 1e6*(1-mask_k), fp32 online softmax, o = P v
//                     (MFMA); the 8 partial (o, max, sum) merge in LDS and
//                     o * sigmoid(g) is written for the output projection.
//   q/k/v/g (one launch, four jobs) and the output projection use linear_rows_kernel
//   (transition.hip).
#include <mutex>

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
    if (hd < H) bias[((long)b * H + hd) * NN + t0 + m] = acc[r] * 1.4426950408889634f;
  }
}

// Attention core: one workgroup of APB_SPLIT waves per (b, head, 32 queries i0 .. i0+31);
// wave w takes key tiles w, w + APB_SPLIT, ... (tiles of 32 keys) and the partial
// results (running max, row sum, unnormalized O) meet in LDS at the end.
// Scores are formed transposed, S^T[key][query] = bias^T + K.Q^T (MFMA, head dim DH
// zero-padded to 32), in log2 units (Q pre-scaled by log2(e)/sqrt(DH), the bias stored
// in log2 units); fp32 online softmax per query (a lane owns one query; its two halves
// hold 16 keys each and meet in one exchange); O^T += V^T P^T (MFMA, P rounded to op_t);
// the merged output is normalized and gated by sigmoid(g).  V^T
// fragments are gathered straight from the fp32 rows: the 32 lanes of a half read 32
// consecutive floats of one key row.
constexpr int APB_SPLIT = 8;
template <int DH>
__global__ __launch_bounds__(64 * APB_SPLIT) void apb_attn_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ g, const float* __restrict__ bias, const float* __restrict__ mask,
    float* __restrict__ og, int B, int N, int n_valid, int c_s, int H, float inf) {
  constexpr float LOG2E_ = 1.4426950408889634f;
  __shared__ float so[APB_SPLIT][32][33];   // [wave][query][d] partial O (padded)
  __shared__ float sm[APB_SPLIT][32], sl[APB_SPLIT][32];
  const int lane = threadIdx.x & 63, h = lane >> 5, m = lane & 31;
  const int wid = threadIdx.x >> 6;
  const int nqb = N / 32;
  const long task = blockIdx.x;
  const int qb = (int)(task % nqb);
  const long bh = task / nqb;
  const int hd = (int)(bh % H), b = (int)(bh / H);
  const int i0 = 32 * qb;
  const float qs = LOG2E_ * rsqrtf((float)DH);
  const long rowb = (long)b * N;
  // Q (B operand): lane (query m, half h), k-step s holds d = 16 s + 8 h + t
  opx8 qf[2];
  {
    const float* qr = q + (rowb + i0 + m) * c_s + hd * DH;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int d = 16 * s2 + 8 * h + t;
        qf[s2][t] = (op_t)(d < DH ? qr[min(d, DH - 1)] * qs : 0.f);
      }
  }
  const float* br = bias + (((long)b * H + hd) * N + i0 + m) * N;   // bias row of query i0 + m
  const float mterm = -inf * LOG2E_;
  f32x16 o = zero16();
  float mref = -INFINITY, lsum = 0.f;
  for (int j0 = 32 * wid; j0 < n_valid; j0 += 32 * APB_SPLIT) {
    // S^T init: bias[q][key] + key mask; register 4g + e is key j0 + 8g + 4h + e
    f32x16 sc;
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const f32x4 bv = *reinterpret_cast<const f32x4*>(br + j0 + 8 * g4 + 4 * h);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = j0 + 8 * g4 + 4 * h + e;
        float t = bv[e];
        if (key >= n_valid) t = -INFINITY;
        else if (mask) t += (1.f - mask[rowb + key]) * mterm;
        sc[4 * g4 + e] = t;
      }
    }
    // K (A operand): lane (key j0 + m, half h), k-step s holds d = 16 s + 8 h + t
    {
      const float* kr = k + (rowb + j0 + m) * c_s + hd * DH;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        opx8 kf;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const int d = 16 * s2 + 8 * h + t;
          kf[t] = (op_t)(d < DH ? kr[min(d, DH - 1)] : 0.f);
        }
        sc = mfma32(kf, qf[s2], sc);
      }
    }
    // online softmax of the tile (fp32); a fully masked prefix keeps mref = -inf, P = 0
    float mx = sc[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sc[r]);
    mx = xor32_max(mx);
    const float mnew = fmaxf(mref, mx);
    const float msub = mnew == -INFINITY ? 0.f : mnew;
    const float alpha = exp2_fast(mref - msub);
    mref = mnew;
    float ps = 0.f;
    opx8 pf[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pr = exp2_fast(sc[r] - msub);
      ps += pr;
      pf[r >> 3][r & 7] = (op_t)pr;
    }
    lsum = lsum * alpha + ps;
#pragma unroll
    for (int r = 0; r < 16; ++r) o[r] *= alpha;
    // V^T (A operand): lane (d = m, half h), k-step ks holds key j0 + 16 ks + 8 (t >> 2) + 4 h + (t & 3)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      opx8 vf;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int key = j0 + 16 * ks + 8 * (t >> 2) + 4 * h + (t & 3);
        vf[t] = (op_t)(m < DH ? v[(rowb + key) * c_s + hd * DH + min(m, DH - 1)] : 0.f);
      }
      o = mfma32(vf, pf[ks], o);
    }
  }
  // partials to LDS: lane (query m, half h) holds o[4 g4 + e] = d 8 g4 + 4 h + e
  const float lw = xor32_sum(lsum);
#pragma unroll
  for (int r = 0; r < 16; ++r) so[wid][m][acc_row(r, h)] = o[r];
  if (h == 0) {
    sm[wid][m] = mref;
    sl[wid][m] = lw;
  }
  __syncthreads();
  // merge: thread t < 32 * DH handles (query t / DH, d t % DH)
  for (int t = threadIdx.x; t < 32 * DH; t += 64 * APB_SPLIT) {
    const int qq = t / DH, d = t - qq * DH;
    float M = -INFINITY;
#pragma unroll
    for (int w2 = 0; w2 < APB_SPLIT; ++w2) M = fmaxf(M, sm[w2][qq]);
    const float Ms = M == -INFINITY ? 0.f : M;
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < APB_SPLIT; ++w2) {
      const float f = exp2_fast(sm[w2][qq] - Ms);
      L += sl[w2][qq] * f;
      O += so[w2][qq][d] * f;
    }
    const long idx = (rowb + i0 + qq) * c_s + hd * DH + d;
    og[idx] = O / L * sigmoidf_fast(g[idx]);
  }
}

// In-place quantize-dequantize of `blocks` consecutive 32-float blocks (MXFP8, fast mode):
// each wave takes 32 blocks, the lane pair (n, n + 32) one block as 16 + 16 values.  Lanes
// past the end compute on block 0 (every lane takes part in the pair exchange) and store
// nothing.
__global__ __launch_bounds__(256) void mx8_fake_quant_rows_kernel(float* __restrict__ x, long blocks) {
  const int lane = threadIdx.x & 63, h = lane >> 5, m = lane & 31;
  const long blk = ((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * 32 + m;
  const bool live = blk < blocks;
  float* p = x + (live ? blk : 0) * 32 + 16 * h;
  f32x16 v;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x4 t = *reinterpret_cast<const f32x4*>(p + 4 * q);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * q + e] = t[e];
  }
  mx_fake_quant16(v);
  if (live) {
#pragma unroll
    for (int q = 0; q < 4; ++q) *reinterpret_cast<f32x4*>(p + 4 * q) = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
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

// Shape / pointer / workspace checks shared by the entry points.
// check_ws = false skips the workspace pointer and size (the allocation-free entry point
// brings its own scratch and checks its size itself).
int pf_apb_check(const pf_apb_args* a, const char* fn, bool bias_only, bool check_ws) {
  if (!a) return pf_fail(PF_E_INVALID, "%s: null args", fn);
  if (a->B <= 0 || a->N <= 0 || a->C != C || a->H <= 0 || a->H > 32 || a->c_s % a->H ||
      (a->c_s / a->H != 24 && a->c_s / a->H != 32) || a->c_s % 32 || a->N > 4096 || (a->N % 32))
    return pf_fail(PF_E_INVALID, "%s: unsupported shape B=%d N=%d c_s=%d C=%d H=%d", fn, a->B, a->N, a->c_s, a->C,
                   a->H);
  if (!a->z || !a->zln_w || !a->zln_b || !a->w_z || (check_ws && !a->workspace))
    return pf_fail(PF_E_INVALID, "%s: null pointer argument", fn);
  if (!bias_only && (!a->s || !a->k_in || !a->out || !a->w_q || !a->b_q || !a->w_k || !a->w_v || !a->w_g ||
                     !a->w_o))
    return pf_fail(PF_E_INVALID, "%s: null pointer argument", fn);
  if (a->n_valid < 0 || a->n_valid > a->N)
    return pf_fail(PF_E_INVALID, "%s: n_valid %d outside [0, N=%d]", fn, a->n_valid, a->N);
  if (!check_ws) return PF_OK;
  const size_t need = pf_apb_workspace_size(a->B, a->N, a->c_s, a->H);
  if (a->workspace_bytes < need)
    return pf_fail(PF_E_INVALID, "%s: workspace too small (%zu < %zu bytes)", fn, a->workspace_bytes, need);
  return PF_OK;
}

// Workspace: q, k, v, g, o*sigmoid(g) [rows][c_s] fp32 each, then the pair bias [B][H][N][N].
float* pf_apb_bias_ptr(const pf_apb_args* a) {
  return (float*)a->workspace + 5 * (size_t)a->B * a->N * a->c_s;
}

int pf_pair_logits(const float* z, const float* lnw, const float* lnb, const void* wz, float* out, int B, int N,
                   int H, float eps, hipStream_t st) {
  const long pairs = (long)B * N * N;
  apb_zbias_kernel<<<(unsigned)((pairs / 32 + 3) / 4), 256, 0, st>>>(z, lnw, lnb, (const op_t*)wz, out, B, N, H, eps);
  PF_CHECK_LAUNCH("apb_zbias_kernel");
  return PF_OK;
}

extern "C" int pf_apb_pair_bias(const pf_apb_args* a) {
  int rc = pf_apb_check(a, "pf_apb_pair_bias", true);
  if (rc) return rc;
  const long pairs = (long)a->B * a->N * a->N;
  apb_zbias_kernel<<<(unsigned)((pairs / 32 + 3) / 4), 256, 0, (hipStream_t)a->stream>>>(
      a->z, a->zln_w, a->zln_b, (const op_t*)a->w_z, pf_apb_bias_ptr(a), a->B, a->N, a->H, a->eps);
  PF_CHECK_LAUNCH("apb_zbias_kernel");
  return PF_OK;
}

namespace {
// fast: o * sigmoid(g) is quantize-dequantized (MXFP8 along c_s) before the output projection.
int apb_attend_impl(const pf_apb_args* a, const char* fn, bool fast) {
  int rc = pf_apb_check(a, fn, false);
  if (rc) return rc;
  const int n_valid = a->n_valid ? a->n_valid : a->N;
  hipStream_t st = (hipStream_t)a->stream;
  const long rows = (long)a->B * a->N;
  const int cs = a->c_s;
  float* q = (float*)a->workspace;
  float* k = q + rows * cs;
  float* v = k + rows * cs;
  float* g = v + rows * cs;
  float* og = g + rows * cs;
  float* bias = pf_apb_bias_ptr(a);
  // q/k/v/g share (rows, c_s, c_s): one launch
  const pf_lin_job proj[4] = {{a->s, a->w_q, nullptr, a->b_q, nullptr, q},
                              {a->k_in, a->w_k, nullptr, nullptr, nullptr, k},
                              {a->k_in, a->w_v, nullptr, nullptr, nullptr, v},
                              {a->s, a->w_g, nullptr, nullptr, nullptr, g}};
  if ((rc = pf_linear_batch(proj, 4, rows, cs, cs, st))) return rc;
  const unsigned grid = (unsigned)((long)a->B * a->H * (a->N / 32));
  if (cs / a->H == 24)
    apb_attn_kernel<24><<<grid, 64 * APB_SPLIT, 0, st>>>(q, k, v, g, bias, a->mask, og, a->B, a->N, n_valid, cs,
                                                        a->H, 1e6f);
  else
    apb_attn_kernel<32><<<grid, 64 * APB_SPLIT, 0, st>>>(q, k, v, g, bias, a->mask, og, a->B, a->N, n_valid, cs,
                                                        a->H, 1e6f);
  PF_CHECK_LAUNCH("apb_attn_kernel");
  if (fast) {
    const long blocks = rows * cs / 32;
    mx8_fake_quant_rows_kernel<<<(unsigned)((blocks + 127) / 128), 256, 0, st>>>(og, blocks);
    PF_CHECK_LAUNCH("mx8_fake_quant_rows_kernel");
  }
  return pf_linear_fwd(og, a->w_o, nullptr, a->accumulate ? a->out : nullptr, a->out, rows, cs, cs, a->stream);
}
}  // namespace

extern "C" int pf_apb_attend(const pf_apb_args* a) { return apb_attend_impl(a, "pf_apb_attend", false); }
extern "C" int pf_apb_attend_mx8(const pf_apb_args* a) { return apb_attend_impl(a, "pf_apb_attend_mx8", true); }

extern "C" int pf_apb_fwd(const pf_apb_args* a) {
  int rc = pf_apb_check(a, "pf_apb_fwd", false);
  if (rc) return rc;
  if ((rc = pf_apb_pair_bias(a))) return rc;
  return pf_apb_attend(a);
}

extern "C" int pf_apb_fwd_mx8(const pf_apb_args* a) {
  int rc = pf_apb_check(a, "pf_apb_fwd_mx8", false);
  if (rc) return rc;
  if ((rc = pf_apb_pair_bias(a))) return rc;
  return pf_apb_attend_mx8(a);
}

// ---------------------------------------------------------------------------------
// pf_apb_fwd without a caller workspace: the scratch (q, k, v, g, o*sigmoid(g) and the pair
// bias, every byte written before it is read) is a file-scope device array.  In host code
// `scratch` only names the symbol: its device address comes from hipGetSymbolAddress, once
// per device with that device current, and only that address is passed to the kernels.
// ---------------------------------------------------------------------------------
constexpr size_t APB_SCRATCH_BYTES = PF_APB_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[APB_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[MAX_DEVICES] = {};   // device address of `scratch` per device

int apb_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
    return pf_fail(PF_E_LAUNCH, "pf_apb_fwd_noalloc: no usable current device (%d)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return pf_fail(PF_E_LAUNCH, "pf_apb_fwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                     hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return PF_OK;
}
}  // namespace

extern "C" int pf_apb_fwd_noalloc(const pf_apb_args* a) {
  // shape, pointers and n_valid first, so an unsupported shape is reported as such
  if (const int rc = pf_apb_check(a, "pf_apb_fwd_noalloc", false, false)) return rc;
  const size_t need = pf_apb_workspace_size(a->B, a->N, a->c_s, a->H);
  if (need > APB_SCRATCH_BYTES)
    return pf_fail(PF_E_INVALID,
                   "pf_apb_fwd_noalloc: B=%d N=%d c_s=%d H=%d needs %zu bytes of scratch, above the static %zu "
                   "(call pf_apb_fwd with a workspace)", a->B, a->N, a->c_s, a->H, need, APB_SCRATCH_BYTES);
  void* ws = nullptr;
  if (const int rc = apb_scratch(&ws)) return rc;
  pf_apb_args b = *a;
  b.workspace = ws;
  b.workspace_bytes = APB_SCRATCH_BYTES;
  return pf_apb_fwd(&b);
}

