// MSA module kernels for gfx950 (Boltz-2 MSALayer minus its no-seq PairformerLayer).
//
// Replaces OuterProductMean.forward (tt_bio/reference.py:596-664) and the ttnn
// OuterProductMean (tt_bio/tenstorrent.py:1632-1720):
//   opm_proj_kernel  LN(m) -> a = W_a, b = W_b (MFMA) * msa_mask, written k-major for the
//                    contraction: At/Bt [B][N*32][S'] (row = (token, channel), k = sequence),
//                    and the mask itself [B][N][S'] for the pair counts.
//   contraction      Z = At . Bt^T  ([B][32N][32N], the einsum "bsic,bsjd->bijcd") and
//                    cnt = M . M^T ([B][N][N], sum_s mask[s,i] mask[s,j]) on the batched
//                    NT kernel of trimul.hip.
//   opm_out_kernel   z[i,j,:] (+)= W_o vec(Z[i,j]) / max(1, cnt[i,j]) + b_o; W_o [128][1024]
//                    streams through LDS by DMA, Z fragments come straight from HBM.
#include "pf_common.h"
#include "pf_internal.h"

namespace {

constexpr int CM = 64;    // c_m (msa_s)
constexpr int CH = 32;    // OPM hidden
constexpr int CZ = 128;   // c_z

// ---------------------------------------------------------------------------------
// OPM projections.  One wave = 32 consecutive sequences s of one token i; lane (s, h)
// holds channels 16 st + 8 h + t (st = 0..3) of its row, so the LayerNorm statistics take
// one lane-half exchange and the values are directly the MFMA B operand.  D[c][s]: lane
// (s, h) holds channels acc_row(r, h) of its sequence and writes them to rows (i, c) of
// the k-major outputs (32 lanes = 64 contiguous bytes per row).
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void opm_proj_kernel(
    const float* __restrict__ m, const float* __restrict__ msa_mask, const float* __restrict__ lnw,
    const float* __restrict__ lnb, const op_t* __restrict__ wa, const op_t* __restrict__ wb,
    op_t* __restrict__ At, op_t* __restrict__ Bt, op_t* __restrict__ Mt, int B, int S, int Sp, int N,
    float eps) {
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, mm = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nsb = Sp / 32;
  const long wv = (long)blockIdx.x * 4 + wid;
  if (wv >= (long)B * N * nsb) return;
  const int sb = (int)(wv % nsb);
  const long bi = wv / nsb;
  const int i = (int)(bi % N), b = (int)(bi / N);
  const int s = 32 * sb + mm;
  const float mk = s < S ? (msa_mask ? msa_mask[((long)b * S + s) * N + i] : 1.f) : 0.f;
  const float* row = m + (((long)b * S + min(s, S - 1)) * N + i) * CM;
  float x[32];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const f32x4 u = *reinterpret_cast<const f32x4*>(row + 16 * st + 8 * h);
    const f32x4 v = *reinterpret_cast<const f32x4*>(row + 16 * st + 8 * h + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[8 * st + e] = u[e];
      x[8 * st + 4 + e] = v[e];
    }
  }
  float sm = 0.f;
#pragma unroll
  for (int k = 0; k < 32; ++k) sm += x[k];
  const float mean = xor32_sum(sm) * (1.f / CM);
  float var = 0.f;
#pragma unroll
  for (int k = 0; k < 32; ++k) { const float d = x[k] - mean; var += d * d; }
  const float rstd = rsqrtf(xor32_sum(var) * (1.f / CM) + eps);
  opx8 xf[4];
#pragma unroll
  for (int st = 0; st < 4; ++st)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int c = 16 * st + 8 * h + t;
      xf[st][t] = (op_t)((x[8 * st + t] - mean) * rstd * lnw[c] + lnb[c]);
    }
  f32x16 ea = zero16(), eb = zero16();
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    ea = mfma32(ld_x8(wa + mm * CM + 16 * st + 8 * h), xf[st], ea);   // rows = channel, cols = sequence
    eb = mfma32(ld_x8(wb + mm * CM + 16 * st + 8 * h), xf[st], eb);
  }
  const long rbase = ((long)b * N + i) * CH * Sp + s;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const long o = rbase + (long)acc_row(r, h) * Sp;
    At[o] = (op_t)(ea[r] * mk);
    Bt[o] = (op_t)(eb[r] * mk);
  }
  if (h == 0) Mt[((long)b * N + i) * Sp + s] = (op_t)mk;
}

// ---------------------------------------------------------------------------------
// OPM output.  A wave owns 32 pairs (i, j0 .. j0+31); the product is D[o][pair] =
// sum_k W_o[o][k] f[pair][k] over k = 32 c + d (1024), 16 chunks of 64 k.  Chunk q of W_o
// ([128][64], 16 KB) arrives by DMA into a 2-stage ring shared by the workgroup's 4 waves
// (rows unpadded, 16-byte chunk c of row R at slot c ^ swz8(R): conflict-free fragment
// reads).  The B operand of k-step u of chunk q is Z[(i, 2q + (u >> 1))][(j, 16 (u & 1) +
// 8 h + t)]: 16 contiguous bytes per lane, loaded one chunk ahead.  The epilogue is the
// output-aligned 16-byte residual update of the pair transition.
// ---------------------------------------------------------------------------------
constexpr int OPM_CHUNK_BYTES = CZ * 64 * 2;   // 16 KB
PF_DEV int swz8r(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }

__global__ __launch_bounds__(256, 2) void opm_out_kernel(
    const op_t* __restrict__ Z, const float* __restrict__ cnt, const op_t* __restrict__ wo,
    const float* __restrict__ bo, float* z, int B, int N, float zscale, int accumulate) {
  __shared__ __attribute__((aligned(16))) char ring[2 * OPM_CHUNK_BYTES];
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, mm = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const long NN = (long)N * N;
  const long p0 = ((long)blockIdx.x * 4 + wid) * 32;   // first pair (b, i, j0); N % 32 == 0
  const bool live = p0 < (long)B * NN;
  const long pc = live ? p0 : 0;                       // idle waves still join every barrier
  const int b = (int)(pc / NN);
  const int i = (int)((pc - (long)b * NN) / N);
  const int j0 = (int)(pc - (long)b * NN - (long)i * N);
  const long ZW = (long)N * CH;                        // row width of Z
  const op_t* zr = Z + ((long)b * ZW + (long)i * CH) * ZW + (long)(j0 + mm) * CH + 8 * h;

  // DMA: wave w moves 1 KB pieces 4w .. 4w+3 (8 rows of 128 bytes each) of a chunk
  uint32_t od[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int R = 8 * (4 * wid + q) + (lane >> 3);
    od[q] = (uint32_t)(2 * (R * 1024 + 8 * ((lane & 7) ^ swz8r(R))));
  }
  auto issue = [&](int q, int buf) PF_INLINE {
    char* st = ring + buf * OPM_CHUNK_BYTES + 4096 * wid;
    const char* src = (const char*)(wo + 64 * q);
#pragma unroll
    for (int u = 0; u < 4; ++u) __builtin_amdgcn_global_load_lds(src + od[u], st + 1024 * u, 16, 0, 0);
  };
  auto zfrag = [&](int q, opx8 (&f)[4]) PF_INLINE {
#pragma unroll
    for (int u = 0; u < 4; ++u) f[u] = ld_x8(zr + (long)(2 * q + (u >> 1)) * ZW + 16 * (u & 1));
  };
  const int sw = swz8r(mm);   // rows 32 ob + m share the low 4 bits of m
  f32x16 acc[4];
#pragma unroll
  for (int ob = 0; ob < 4; ++ob) acc[ob] = zero16();
  opx8 fz[4], fn[4];
  issue(0, 0);
  zfrag(0, fn);
  for (int q = 0; q < 16; ++q) {
    __builtin_amdgcn_s_waitcnt(vmcnt_le(0));   // chunk q and its Z fragments landed ...
    __builtin_amdgcn_s_barrier();              // ... for every wave; the other stage is free
    asm volatile("" ::: "memory");
#pragma unroll
    for (int u = 0; u < 4; ++u) fz[u] = fn[u];
    if (q + 1 < 16) {
      issue(q + 1, (q + 1) & 1);
      zfrag(q + 1, fn);
    }
    const char* st = ring + (q & 1) * OPM_CHUNK_BYTES;
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) {
      const char* wrow = st + (32 * ob + mm) * 128;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const opx8 wf = *reinterpret_cast<const opx8*>(wrow + 16 * ((2 * u + h) ^ sw));
        acc[ob] = mfma32(wf, fz[u], acc[ob]);   // rows = output channel, cols = pair
      }
    }
  }
  if (!live) return;
  // lane (pair m, h): acc[ob][4 g + e] is channel 32 ob + 8 g + 4 h + e
  const long p = p0 + mm;
  const float sc = zscale / fmaxf(cnt[(long)b * NN + (long)i * N + j0 + mm], 1.f);
  float* dst = z + p * CZ;
  f32x4 res[16];
#pragma unroll
  for (int q = 0; q < 16; ++q)
    res[q] = accumulate ? *reinterpret_cast<const f32x4*>(dst + oa_channel(q, h)) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const f32x4 bb = *reinterpret_cast<const f32x4*>(bo + oa_channel(q, h));
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = acc[q >> 2][4 * (q & 3) + e] * sc + bb[e] + res[q][e];
    *reinterpret_cast<f32x4*>(dst + oa_channel(q, h)) = v;
  }
}

}  // namespace

// Workspace of pf_opm_fwd: At, Bt [B][32N][S'], mask [B][N][S'], Z [B][32N][32N] (op_t),
// cnt [B][N][N] (fp32); S' = S rounded up to 64.
extern "C" size_t pf_opm_workspace_size(int B, int S, int N) {
  if (B <= 0 || S <= 0 || N <= 0) return 0;
  const size_t Sp = (size_t)(S + 63) / 64 * 64;
  const size_t rows = (size_t)B * N * CH;
  return (2 * rows * Sp + (size_t)B * N * Sp + rows * N * CH) * sizeof(op_t) + (size_t)B * N * N * sizeof(float);
}

extern "C" int pf_opm_fwd(const pf_opm_args* a) {
  if (!a) return pf_fail(PF_E_INVALID, "pf_opm_fwd: null args");
  if (a->c_m != CM || a->c_hidden != CH || a->C != CZ)
    return pf_fail(PF_E_INVALID, "pf_opm_fwd: need c_m = 64, c_hidden = 32, C = 128 (got %d, %d, %d)", a->c_m,
                   a->c_hidden, a->C);
  if (a->B <= 0 || a->S <= 0 || a->N <= 0 || a->N % 32)
    return pf_fail(PF_E_INVALID, "pf_opm_fwd: need B, S > 0 and N a positive multiple of 32 (B=%d S=%d N=%d)", a->B,
                   a->S, a->N);
  if ((long)a->N * CH * ((a->S + 63) / 64 * 64) >= (1l << 31) || (long)a->B * a->N * a->N >= (1l << 31))
    return pf_fail(PF_E_INVALID, "pf_opm_fwd: shape too large (B=%d S=%d N=%d)", a->B, a->S, a->N);
  if (!a->m || !a->z || !a->norm_w || !a->norm_b || !a->w_a || !a->w_b || !a->w_o || !a->b_o || !a->workspace)
    return pf_fail(PF_E_INVALID, "pf_opm_fwd: null pointer argument");
  const size_t need = pf_opm_workspace_size(a->B, a->S, a->N);
  if (a->workspace_bytes < need)
    return pf_fail(PF_E_INVALID, "pf_opm_fwd: workspace too small (%zu < %zu bytes)", a->workspace_bytes, need);
  hipStream_t st = (hipStream_t)a->stream;
  const int B = a->B, S = a->S, N = a->N, Sp = (S + 63) / 64 * 64;
  const size_t rows = (size_t)B * N * CH;
  op_t* At = (op_t*)a->workspace;
  op_t* Bt = At + rows * Sp;
  op_t* Mt = Bt + rows * Sp;
  op_t* Z = Mt + (size_t)B * N * Sp;
  float* cnt = (float*)(Z + rows * N * CH);
  const long waves = (long)B * N * (Sp / 32);
  opm_proj_kernel<<<(unsigned)((waves + 3) / 4), 256, 0, st>>>(a->m, a->msa_mask, a->norm_w, a->norm_b,
                                                              (const op_t*)a->w_a, (const op_t*)a->w_b, At, Bt, Mt,
                                                              B, S, Sp, N, a->eps);
  PF_CHECK_LAUNCH("opm_proj_kernel");
  int rc = pf_contract_rect(At, Bt, Z, 0, B, N * CH, N * CH, Sp, X_STORE_SCALE, st);
  if (rc) return rc;
  if ((rc = pf_contract_rect(Mt, Mt, cnt, 1, B, N, N, Sp, 1.f, st))) return rc;
  const long pairs = (long)B * N * N;
  opm_out_kernel<<<(unsigned)((pairs / 32 + 3) / 4), 256, 0, st>>>(Z, cnt, (const op_t*)a->w_o, a->b_o, a->z, B, N,
                                                                  X_LOAD_SCALE, a->accumulate);
  PF_CHECK_LAUNCH("opm_out_kernel");
  return PF_OK;
}
