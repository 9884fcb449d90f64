// Triangle attention (starting / ending node) for gfx950.
//
// Replaces TriangleAttention.forward (tt_bio/reference.py:294-365 with Attention
// 33-194, _attention tt_bio/boltz2.py:790-810, chunk_layer 542-628) and the ttnn
// TriangleAttention (tt_bio/tenstorrent.py:506-650).
//
// "Frame" coordinates: the starting node attends along rows of z, the ending node
// along rows of z^T.  Frame pair (i, j) is z pair (i, j) (starting) or (j, i)
// (ending); transposition is done by addressing, never materialized.
//
//   ta_proj  LN(z) -> q (pre-scaled by log2(e)/sqrt(d)), k, v^T, per-head bias
//            (x log2(e)) and the per-(row, key) additive mask term, one pass over z.
//              Q, K  bf16 [B][N(row i)][H][N(j)][D]
//              Vt    bf16 [B][N(row i)][H][D][N(k)]
//              bias2 fp32 [B][H][N(j)][N(k)]   (shared by all rows i)
//              M2    fp32 [B][N(i)][N(k)]      1e9*(mask-1)*log2(e)
//   ta_attn  one workgroup per (b, row i, 64 queries), one wave per head.  Works in
//            the transposed score layout S^T[key][query] so each lane owns one query:
//            the bias tile is loaded straight into the MFMA accumulator, the online
//            softmax statistics are per lane (plus one cross-half exchange), and the
//            probabilities feed the P.V MFMA from registers via the k-permutation
//            described in pf_common.h.  Epilogue (fused mode): gate recomputed from
//            LN(z), o * sigmoid(g) -> LDS -> linear_o -> residual into z.
#include "pf_common.h"
#include "pf_internal.h"

namespace {

constexpr int C = 128, H = 4, D = 32, LDSW = 136;
constexpr float LOG2E = 1.4426950408889634f;

struct Blk32 { bf16x8 v[2]; };
// Load rows [0, nrows) of a [*][128] bf16 block (rows >= nrows read as zero).
PF_DEV void blk32_load(const bf16* __restrict__ src, int nrows, int tid, Blk32& r) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int c = tid + 256 * q;
    const int row = c >> 4;
    if (row < nrows) {
      r.v[q] = ld_bf16x8(src + row * C + (c & 15) * 8);
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) r.v[q][t] = (bf16)0.f;
    }
  }
}
PF_DEV void blk32_store(bf16* lds, int tid, const Blk32& r) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int c = tid + 256 * q;
    *reinterpret_cast<bf16x8*>(lds + (c >> 4) * LDSW + (c & 15) * 8) = r.v[q];
  }
}

// ---------------------------------------------------------------------------------
// Projection: one wave = 32 frame positions (ip, j0 .. j0+31).
// Weight blocks (32 rows each): 0-3 q heads, 4-7 k heads, 8-11 v heads, 12 bias.
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ta_proj_kernel(
    const float* __restrict__ z, const float* __restrict__ pair_mask,
    const float* __restrict__ lnw, const float* __restrict__ lnb,
    const bf16* __restrict__ wq, const bf16* __restrict__ wk, const bf16* __restrict__ wv,
    const bf16* __restrict__ wb, bf16* __restrict__ Q, bf16* __restrict__ K,
    bf16* __restrict__ Vt, float* __restrict__ bias2, float* __restrict__ M2,
    int B, int N, int ending, float qscale, float eps) {
  __shared__ __attribute__((aligned(16))) bf16 lds[2][32 * LDSW];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, h = lane >> 5, m = lane & 31;
  const long NN = (long)N * N;
  const long pos0 = ((long)blockIdx.x * 4 + wid) * 32;
  const bool active = pos0 < (long)B * NN;

  int b = 0, ip = 0, j0 = 0;
  bf16x8 xf[8];
  if (active) {
    b = (int)(pos0 / NN);
    const long t0 = pos0 - (long)b * NN;
    ip = (int)(t0 / N);
    j0 = (int)(t0 - (long)ip * N);
    const int zi = ending ? j0 + m : ip;
    const int zj = ending ? ip : j0 + m;
    const long pair = ((long)b * N + zi) * N + zj;
    float x[64];
    load_row128_frag(z + pair * C, h, x);
    ln128_to_frag(x, h, lnw, lnb, eps, xf);
    if (h == 0) {
      const float mv = pair_mask ? pair_mask[pair] : 1.f;
      M2[((long)b * N + ip) * N + j0 + m] = 1e9f * (mv - 1.f) * LOG2E;
    }
  }

  auto src = [&](int bk) -> const bf16* {
    return bk < 4 ? wq + bk * 32 * C : bk < 8 ? wk + (bk - 4) * 32 * C
         : bk < 12 ? wv + (bk - 8) * 32 * C : wb;
  };
  Blk32 rw;
  blk32_load(src(0), 32, tid, rw);
  for (int bk = 0; bk < 13; ++bk) {
    bf16* lw = lds[bk & 1];
    blk32_store(lw, tid, rw);
    __syncthreads();
    if (bk + 1 < 13) blk32_load(src(bk + 1), bk + 1 < 12 ? 32 : H, tid, rw);
    if (!active) continue;
    f32x16 acc = zero16();
    if (bk < 8) {
      // normal orientation: rows = positions, cols = head dim
#pragma unroll
      for (int s = 0; s < 8; ++s) acc = mfma32(xf[s], ld_bf16x8(lw + m * LDSW + 16 * s + 8 * h), acc);
      bf16* dst = bk < 4 ? Q : K;
      const float sc = bk < 4 ? qscale : 1.f;
      const long base = ((((long)b * N + ip) * H + (bk & 3)) * N + j0) * D;
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[base + acc_row(r, h) * D + m] = (bf16)(acc[r] * sc);
    } else {
      // transposed orientation: rows = head dim (or head for the bias), cols = positions
#pragma unroll
      for (int s = 0; s < 8; ++s) acc = mfma32(ld_bf16x8(lw + m * LDSW + 16 * s + 8 * h), xf[s], acc);
      if (bk < 12) {
        const long base = (((long)b * N + ip) * H + (bk - 8)) * D * (long)N + j0 + m;
#pragma unroll
        for (int r = 0; r < 16; ++r) Vt[base + (long)acc_row(r, h) * N] = (bf16)acc[r];
      } else if (h == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) bias2[(((long)b * H + r) * N + ip) * N + j0 + m] = acc[r] * LOG2E;
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Flash attention.  FUSED: gate + linear_o + residual into z.  Otherwise write o.
// ---------------------------------------------------------------------------------
template <bool FUSED>
__global__ __launch_bounds__(256, 2) void ta_attn_kernel(
    const bf16* __restrict__ Q, const bf16* __restrict__ K, const bf16* __restrict__ Vt,
    const float* __restrict__ bias2, const float* __restrict__ M2,
    const float* z_in, float* out, const float* __restrict__ lnw, const float* __restrict__ lnb,
    const bf16* __restrict__ wg, const bf16* __restrict__ wo, float* __restrict__ O,
    int N, int ending, int accumulate, float eps, int total) {
  __shared__ __attribute__((aligned(16))) bf16 sX[FUSED ? 64 * LDSW : 8];
  __shared__ __attribute__((aligned(16))) bf16 sO[FUSED ? 64 * LDSW : 8];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, h = lane >> 5, m = lane & 31;
  const int nJB = N / 64;
  const int w = xcd_remap(blockIdx.x, total);
  const int b = w / (N * nJB);
  const int rem = w - b * N * nJB;
  const int ip = rem / nJB;
  const int j0 = (rem - ip * nJB) * 64;
  const long NN = (long)N * N;

  if (FUSED && wid < 2) {
    // LN(z) of the 64 frame pairs, for the gate; waves 0/1 take 32 positions each.
    const int j = j0 + 32 * wid + m;
    const long pair = ending ? ((long)b * N + j) * N + ip : ((long)b * N + ip) * N + j;
    float x[64];
    bf16x8 xf[8];
    load_row128_frag(z_in + pair * C, h, x);
    ln128_to_frag(x, h, lnw, lnb, eps, xf);
#pragma unroll
    for (int s = 0; s < 8; ++s)
      *reinterpret_cast<bf16x8*>(&sX[(32 * wid + m) * LDSW + 16 * s + 8 * h]) = xf[s];
  }

  const long rowbase = ((long)b * N + ip) * H + wid;
  const bf16* Qh = Q + rowbase * N * D;
  const bf16* Kh = K + rowbase * N * D;
  const bf16* Vh = Vt + rowbase * D * N;
  const float* Bh = bias2 + ((long)b * H + wid) * NN;
  const float* Mr = M2 + ((long)b * N + ip) * N;

  bf16x8 qf[2][2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int s = 0; s < 2; ++s) qf[qb][s] = ld_bf16x8(Qh + (long)(j0 + 32 * qb + m) * D + 16 * s + 8 * h);

  f32x16 o[2] = {zero16(), zero16()};
  float mrun[2] = {-INFINITY, -INFINITY}, lrun[2] = {0.f, 0.f};

  for (int kb0 = 0; kb0 < N; kb0 += 64) {
    f32x16 sc[2][2];   // [key block][query block], S^T: rows = keys, cols = queries
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const float* bp = Bh + (long)(j0 + 32 * qb + m) * N + kb0 + 32 * kb + 4 * h;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 bv = *reinterpret_cast<const f32x4*>(bp + 8 * g);
          sc[kb][qb][4 * g + 0] = bv[0]; sc[kb][qb][4 * g + 1] = bv[1];
          sc[kb][qb][4 * g + 2] = bv[2]; sc[kb][qb][4 * g + 3] = bv[3];
        }
      }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const bf16x8 kf = ld_bf16x8(Kh + (long)(kb0 + 32 * kb + m) * D + 16 * s + 8 * h);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) sc[kb][qb] = mfma32(kf, qf[qb][s], sc[kb][qb]);
      }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 mv = *reinterpret_cast<const f32x4*>(Mr + kb0 + 32 * kb + 8 * g + 4 * h);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          sc[kb][qb][4 * g + 0] += mv[0]; sc[kb][qb][4 * g + 1] += mv[1];
          sc[kb][qb][4 * g + 2] += mv[2]; sc[kb][qb][4 * g + 3] += mv[3];
        }
      }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      float mx = sc[0][qb][0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sc[0][qb][r]);
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[1][qb][r]);
      mx = xor32_max(mx);
      const float mnew = fmaxf(mrun[qb], mx);
      const float alpha = exp2_fast(mrun[qb] - mnew);
      mrun[qb] = mnew;
      float ps = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = exp2_fast(sc[kb][qb][r] - mnew);
          sc[kb][qb][r] = p;
          ps += p;
        }
      lrun[qb] = lrun[qb] * alpha + ps;
#pragma unroll
      for (int r = 0; r < 16; ++r) o[qb][r] *= alpha;
    }
    // O^T[d][q] += V^T[d][keys] * P^T[keys][q], keys in the accumulator's k-permutation
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16* vp = Vh + (long)m * N + kb0 + 32 * kb + 16 * ks + 4 * h;
        const bf16x8 vf = cat44(ld_bf16x4(vp), ld_bf16x4(vp + 8));
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          bf16x8 pf;
#pragma unroll
          for (int t = 0; t < 8; ++t) pf[t] = (bf16)sc[kb][qb][8 * ks + t];
          o[qb] = mfma32(vf, pf, o[qb]);
        }
      }
  }

#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float inv = 1.f / xor32_sum(lrun[qb]);
#pragma unroll
    for (int r = 0; r < 16; ++r) o[qb][r] *= inv;
  }

  if (!FUSED) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        O[(rowbase * N + j0 + 32 * qb + m) * D + acc_row(r, h)] = o[qb][r];
    return;
  }

  __syncthreads();   // sX ready
  // gate^T for this head: rows = head dim, cols = queries (same layout as o)
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    f32x16 g = zero16();
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const bf16x8 wf = ld_bf16x8(wg + (32 * wid + m) * C + 16 * s + 8 * h);
      const bf16x8 xf = ld_bf16x8(&sX[(32 * qb + m) * LDSW + 16 * s + 8 * h]);
      g = mfma32(wf, xf, g);
    }
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      bf16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (bf16)(o[qb][4 * g4 + e] * sigmoidf_fast(g[4 * g4 + e]));
      *reinterpret_cast<bf16x4*>(&sO[(32 * qb + m) * LDSW + 32 * wid + 8 * g4 + 4 * h]) = v;
    }
  }
  __syncthreads();   // sO ready
  // linear_o: wave `wid` produces output channels [32*wid, 32*wid + 32)
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    f32x16 acc = zero16();
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const bf16x8 of = ld_bf16x8(&sO[(32 * qb + m) * LDSW + 16 * s + 8 * h]);
      const bf16x8 wf = ld_bf16x8(wo + (32 * wid + m) * C + 16 * s + 8 * h);
      acc = mfma32(of, wf, acc);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int j = j0 + 32 * qb + acc_row(r, h);
      const long pair = ending ? ((long)b * N + j) * N + ip : ((long)b * N + ip) * N + j;
      const long idx = pair * C + 32 * wid + m;
      out[idx] = accumulate ? out[idx] + acc[r] : acc[r];
    }
  }
}

// Layout conversion for the standalone attention core (fp32 API tensors -> kernel layout).
__global__ void ta_prep_qkv_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                   const float* __restrict__ v, float qs, bf16* __restrict__ Q,
                                   bf16* __restrict__ K, bf16* __restrict__ Vt, long rows, int N) {
  // rows = B*N*H sequences of N x D; element e of sequence r: (j, d) = (e / D, e % D)
  const long total = rows * N * D;
  for (long e = (long)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (long)gridDim.x * blockDim.x) {
    const long r = e / ((long)N * D);
    const int jd = (int)(e - r * N * D);
    const int j = jd / D, d = jd - j * D;
    Q[e] = (bf16)(q[e] * qs);
    K[e] = (bf16)k[e];
    Vt[r * N * D + (long)d * N + j] = (bf16)v[e];
  }
}

__global__ void ta_prep_bias_kernel(const float* __restrict__ bias, const float* __restrict__ mask,
                                    float* __restrict__ bias2, float* __restrict__ M2,
                                    long nbias, long nmask) {
  for (long e = (long)blockIdx.x * blockDim.x + threadIdx.x; e < nbias; e += (long)gridDim.x * blockDim.x) {
    bias2[e] = bias[e] * LOG2E;
    if (e < nmask) M2[e] = mask ? 1e9f * (mask[e] - 1.f) * LOG2E : 0.f;
  }
}

struct TaBuffers {
  bf16 *Q, *K, *Vt;
  float *bias2, *M2;
};

size_t ta_buffers_size(int B, int N) {
  const size_t e = (size_t)B * N * H * N * D;
  return 3 * e * sizeof(bf16) + ((size_t)B * H * N * N + (size_t)B * N * N) * sizeof(float);
}

TaBuffers ta_buffers(void* ws, int B, int N) {
  const size_t e = (size_t)B * N * H * N * D;
  TaBuffers t;
  t.Q = (bf16*)ws;
  t.K = t.Q + e;
  t.Vt = t.K + e;
  t.bias2 = (float*)(t.Vt + e);
  t.M2 = t.bias2 + (size_t)B * H * N * N;
  return t;
}

}  // namespace

// ---------------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------------
extern "C" size_t pf_triatt_workspace_size(int B, int N, int C_, int H_, int D_) {
  if (B <= 0 || N <= 0 || C_ != C || H_ != H || D_ != D) return 0;
  return ta_buffers_size(B, N);
}

extern "C" int pf_triatt_fwd(const pf_triatt_args* a) {
  if (!a) return pf_fail(PF_E_INVALID, "pf_triatt_fwd: null args");
  if (a->C != C || a->H != H || a->D != D)
    return pf_fail(PF_E_INVALID, "pf_triatt_fwd: only C=128, H=4, D=32 supported (got C=%d H=%d D=%d)",
                   a->C, a->H, a->D);
  if (a->B <= 0 || a->N <= 0 || a->N % 64)
    return pf_fail(PF_E_INVALID, "pf_triatt_fwd: need B > 0 and N a positive multiple of 64 (B=%d N=%d)", a->B, a->N);
  if (!a->z_in || !a->out || !a->ln_w || !a->ln_b || !a->w_bias || !a->w_q || !a->w_k ||
      !a->w_v || !a->w_g || !a->w_o || !a->workspace)
    return pf_fail(PF_E_INVALID, "pf_triatt_fwd: null pointer argument");
  const size_t need = ta_buffers_size(a->B, a->N);
  if (a->workspace_bytes < need)
    return pf_fail(PF_E_INVALID, "pf_triatt_fwd: workspace too small (%zu < %zu bytes)", a->workspace_bytes, need);
  hipStream_t st = (hipStream_t)a->stream;
  const int B = a->B, N = a->N;
  TaBuffers t = ta_buffers(a->workspace, B, N);
  const float qscale = LOG2E / sqrtf((float)D);
  const long positions = (long)B * N * N;
  const int grid_proj = (int)((positions / 32 + 3) / 4);
  ta_proj_kernel<<<grid_proj, 256, 0, st>>>(a->z_in, a->pair_mask, a->ln_w, a->ln_b,
                                            (const bf16*)a->w_q, (const bf16*)a->w_k, (const bf16*)a->w_v,
                                            (const bf16*)a->w_bias, t.Q, t.K, t.Vt, t.bias2, t.M2, B, N,
                                            a->ending, qscale, a->eps);
  PF_CHECK_LAUNCH("ta_proj_kernel");
  const int total = B * N * (N / 64);
  ta_attn_kernel<true><<<total, 256, 0, st>>>(t.Q, t.K, t.Vt, t.bias2, t.M2, a->z_in, a->out, a->ln_w,
                                              a->ln_b, (const bf16*)a->w_g, (const bf16*)a->w_o, nullptr,
                                              N, a->ending, a->accumulate, a->eps, total);
  PF_CHECK_LAUNCH("ta_attn_kernel");
  return PF_OK;
}

extern "C" size_t pf_tri_attention_workspace_size(int B, int N, int H_, int D_) {
  if (B <= 0 || N <= 0 || H_ != H || D_ != D) return 0;
  return ta_buffers_size(B, N);
}

extern "C" int pf_tri_attention(const float* q, const float* k, const float* v, const float* bias,
                                const float* mask, float scale, float* o, int B, int N, int H_, int D_,
                                void* workspace, size_t workspace_bytes, void* stream) {
  if (H_ != H || D_ != D)
    return pf_fail(PF_E_INVALID, "pf_tri_attention: only H=4, D=32 supported (got H=%d D=%d)", H_, D_);
  if (B <= 0 || N <= 0 || N % 64)
    return pf_fail(PF_E_INVALID, "pf_tri_attention: need B > 0 and N a positive multiple of 64 (B=%d N=%d)", B, N);
  if (!q || !k || !v || !bias || !o || !workspace)
    return pf_fail(PF_E_INVALID, "pf_tri_attention: null pointer argument");
  const size_t need = ta_buffers_size(B, N);
  if (workspace_bytes < need)
    return pf_fail(PF_E_INVALID, "pf_tri_attention: workspace too small (%zu < %zu bytes)", workspace_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  TaBuffers t = ta_buffers(workspace, B, N);
  const long rows = (long)B * N * H;
  ta_prep_qkv_kernel<<<2048, 256, 0, st>>>(q, k, v, scale * LOG2E, t.Q, t.K, t.Vt, rows, N);
  PF_CHECK_LAUNCH("ta_prep_qkv_kernel");
  ta_prep_bias_kernel<<<1024, 256, 0, st>>>(bias, mask, t.bias2, t.M2, (long)B * H * N * N, (long)B * N * N);
  PF_CHECK_LAUNCH("ta_prep_bias_kernel");
  const int total = B * N * (N / 64);
  ta_attn_kernel<false><<<total, 256, 0, st>>>(t.Q, t.K, t.Vt, t.bias2, t.M2, nullptr, nullptr, nullptr,
                                               nullptr, nullptr, nullptr, o, N, 0, 0, 0.f, total);
  PF_CHECK_LAUNCH("ta_attn_kernel");
  return PF_OK;
}
