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

// ---------------------------------------------------------------------------------
// Pair weighted averaging (PairWeightedAveraging.forward, tt_bio/reference.py:715-790):
//   logits   log2(e) * LN_z(z) . W_z[h] by the single track's pair-bias kernel
//   softmax  pwa_softmax_kernel: over j, with -1e6 * (1 - mask[i,j]), to fp16 weights
//            Wt [B*H][N (i)][N (j)]
//   v        pwa_proj_kernel: W_m LN_m(m) written k-major, v_t [B*H][S*32 (s, d)][N (j)]
//   average  O[b*H+h][i][(s, d)] = sum_j Wt[.][i][j] v_t[.][(s, d)][j] on the batched NT
//            kernel ("bhij,bhsjd->bhsid")
//   output   pwa_out_kernel: gate sigmoid(W_g LN_m(m)) recomputed in registers, times O,
//            W_o (64 x 256), residual into m
// ---------------------------------------------------------------------------------
constexpr int PH = 8, PD = 32, PHD = PH * PD;   // heads, head width, 256

// One wave per row (b, h, i): three passes over the row (max, sum, write).
__global__ __launch_bounds__(256) void pwa_softmax_kernel(const float* __restrict__ logits,
                                                          const float* __restrict__ pair_mask, op_t* __restrict__ Wt,
                                                          int B, int N) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= (long)B * PH * N) return;
  const int i = (int)(row % N);
  const int b = (int)(row / ((long)PH * N));
  const float* x = logits + row * N;
  const float* pm = pair_mask ? pair_mask + ((long)b * N + i) * N : nullptr;
  constexpr float MASKED = -1e6f * 1.4426950408889634f;   // reference -inf = 1e6, log2 units
  auto val = [&](int j) PF_INLINE { return x[j] + (pm ? (1.f - pm[j]) * MASKED : 0.f); };
  float mx = -INFINITY;
  for (int j = lane; j < N; j += 64) mx = fmaxf(mx, val(j));
  mx = wave_max(mx);
  float sm = 0.f;
  for (int j = lane; j < N; j += 64) sm += exp2_fast(val(j) - mx);
  const float inv = 1.f / wave_sum(sm);
  op_t* w = Wt + row * N;
  for (int j = lane; j < N; j += 64) w[j] = (op_t)(exp2_fast(val(j) - mx) * inv);
}

// v projection: a wave takes 32 consecutive tokens j of one (b, s); W_m [256][64] sits in
// LDS (128-byte rows, 16-byte chunk c of row R at slot c ^ swz8r(R)).  D[(h, d)][j]: lane
// (j, half) writes v_t rows ((b*H + h)*S + s)*32 + d at column j (64 contiguous bytes per
// row and register).
__global__ __launch_bounds__(512) void pwa_proj_kernel(
    const float* __restrict__ m, const float* __restrict__ lnw, const float* __restrict__ lnb,
    const op_t* __restrict__ wm, op_t* __restrict__ vt, int B, int S, int N, float eps) {
  __shared__ __attribute__((aligned(16))) op_t sw[PHD * CM];
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, mm = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  for (int c = tid; c < PHD * 8; c += 512) {
    const int R = c >> 3, k = c & 7;
    st_x8(sw + R * CM + 8 * (k ^ swz8r(R)), ld_x8(wm + R * CM + 8 * k));
  }
  __syncthreads();
  const int nj = N / 32;
  const long wv = (long)blockIdx.x * 8 + wid;
  if (wv >= (long)B * S * nj) return;
  const int j0 = 32 * (int)(wv % nj);
  const long bs = wv / nj;   // b * S + s
  const int s = (int)(bs % S), b = (int)(bs / S);
  opx8 xf[4];
  ln64_to_frag(m + (bs * N + j0 + mm) * CM, h, lnw, lnb, eps, xf);
  const int sw8 = swz8r(mm);
#pragma unroll 1
  for (int blk = 0; blk < PH; ++blk) {
    f32x16 acc = zero16();
#pragma unroll
    for (int st = 0; st < 4; ++st)
      acc = mfma32(ld_x8(sw + (32 * blk + mm) * CM + 8 * ((2 * st + h) ^ sw8)), xf[st], acc);   // rows = (h, d)
    op_t* dst = vt + (((long)b * PH + blk) * S + s) * PD * (long)N + j0 + mm;
#pragma unroll
    for (int r = 0; r < 16; ++r) dst[(long)acc_row(r, h) * N] = (op_t)acc[r];
  }
}

// Output: a wave takes 32 consecutive sequences s of one (b, i).  W_g [256][64] and
// W_o [64][256] sit in LDS.  The gate is formed as D[k][s] with W_g rows loaded in perm16
// order, so its accumulator registers 8 s' + t of half h hold k = 16 s' + 8 h + t of the
// block -- the B-operand order of the W_o product; each such fragment is multiplied by
// the matching 16 bytes of O and fed to D[o][s] += W_o . og.  Residual into m in the
// output-aligned layout (16-byte loads / stores).
__global__ __launch_bounds__(512) void pwa_out_kernel(
    const float* m_in, float* m_out, const float* __restrict__ lnw, const float* __restrict__ lnb,
    const op_t* __restrict__ wg, const op_t* __restrict__ wo, const op_t* __restrict__ O, int B, int S, int N,
    int accumulate, float eps) {
  __shared__ __attribute__((aligned(16))) op_t sg[PHD * CM];
  __shared__ __attribute__((aligned(16))) op_t so[CM * PHD];
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, mm = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  for (int c = tid; c < PHD * 8; c += 512) {   // W_g: 256 rows of 8 chunks
    const int R = c >> 3, k = c & 7;
    st_x8(sg + R * CM + 8 * (k ^ swz8r(R)), ld_x8(wg + R * CM + 8 * k));
  }
  for (int c = tid; c < CM * 32; c += 512) {   // W_o: 64 rows of 32 chunks
    const int R = c >> 5, k = c & 31;
    st_x8(so + R * PHD + 8 * (k ^ (R & 15)), ld_x8(wo + R * PHD + 8 * k));
  }
  __syncthreads();
  const int ns = (S + 31) / 32;
  const long wv = (long)blockIdx.x * 8 + wid;
  if (wv >= (long)B * N * ns) return;
  const int s0 = 32 * (int)(wv % ns);
  const long bi = wv / ns;   // b * N + i
  const int i = (int)(bi % N), b = (int)(bi / N);
  const int s = min(s0 + mm, S - 1);   // rows past S are computed on a clamped row and not stored
  const long mrow = (((long)b * S + s) * N + i) * CM;
  opx8 xf[4];
  ln64_to_frag(m_in + mrow, h, lnw, lnb, eps, xf);
  const int gr = perm16(mm), sg8 = swz8r(gr);
  f32x16 acc[2] = {zero16(), zero16()};
#pragma unroll 1
  for (int blk = 0; blk < PH; ++blk) {
    f32x16 g = zero16();
#pragma unroll
    for (int st = 0; st < 4; ++st)
      g = mfma32(ld_x8(sg + (32 * blk + gr) * CM + 8 * ((2 * st + h) ^ sg8)), xf[st], g);   // rows = k (perm16)
    const op_t* orow = O + ((long)(b * PH + blk) * N + i) * ((long)S * PD) + (long)s * PD + 8 * h;
#pragma unroll
    for (int sp = 0; sp < 2; ++sp) {
      const opx8 ov = ld_x8(orow + 16 * sp);
      opx8 og;
#pragma unroll
      for (int t = 0; t < 8; ++t) og[t] = (op_t)((float)ov[t] * sigmoidf_fast(g[8 * sp + t]));
      const int kc = 2 * (2 * blk + sp) + h;   // 16-byte chunk of the W_o row: k = 32 blk + 16 sp + 8 h
#pragma unroll
      for (int ob = 0; ob < 2; ++ob) {
        const int R = 32 * ob + mm;
        acc[ob] = mfma32(ld_x8(so + R * PHD + 8 * (kc ^ (R & 15))), og, acc[ob]);   // rows = output channel
      }
    }
  }
  if (s0 + mm >= S) return;
  // lane (s, h): acc[ob][4 g + e] is channel 32 ob + 8 g + 4 h + e
  const float* src = m_in + mrow;
  float* dst = m_out + mrow;
  f32x4 res[8];
#pragma unroll
  for (int q = 0; q < 8; ++q)
    res[q] = accumulate ? *reinterpret_cast<const f32x4*>(src + oa_channel(q, h)) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = acc[q >> 2][4 * (q & 3) + e] + res[q][e];
    *reinterpret_cast<f32x4*>(dst + oa_channel(q, h)) = v;
  }
}

// ---------------------------------------------------------------------------------
// MSA input embedding (MSAModule.forward, tt_bio/reference.py:1253-1276):
//   m[b,s,i,:] = W[:, msa[b,s,i]] + has_del W[:,T] + del_val W[:,T+1] + paired W[:,T+2]
//                + s_emb[b,i,:]
// the one-hot product as a column gather; one thread per 4 channels.
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void msa_embed_kernel(
    const int* __restrict__ msa, const float* __restrict__ has_del, const float* __restrict__ del_val,
    const float* __restrict__ paired, const float* __restrict__ s_emb, const float* __restrict__ wt,
    float* __restrict__ m, long rows, int S, int N, int n_tok) {
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= rows * (CM / 4)) return;
  const long r = t / (CM / 4);
  const int c0 = 4 * (int)(t - r * (CM / 4));
  const int i = (int)(r % N);
  const long b = r / ((long)S * N);
  const int tok = min(max(msa[r], 0), n_tok - 1);
  const float f0 = has_del ? has_del[r] : 0.f, f1 = del_val ? del_val[r] : 0.f, f2 = paired ? paired[r] : 0.f;
  // wt is the transposed projection [n_tok + 3][CM]: one row per input feature
  const f32x4 e = *reinterpret_cast<const f32x4*>(s_emb + (b * N + i) * CM + c0);
  const f32x4 w0 = *reinterpret_cast<const f32x4*>(wt + (long)tok * CM + c0);
  const f32x4 w1 = *reinterpret_cast<const f32x4*>(wt + (long)n_tok * CM + c0);
  const f32x4 w2 = *reinterpret_cast<const f32x4*>(wt + (long)(n_tok + 1) * CM + c0);
  const f32x4 w3 = *reinterpret_cast<const f32x4*>(wt + (long)(n_tok + 2) * CM + c0);
  f32x4 v;
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = w0[k] + f0 * w1[k] + f1 * w2[k] + f2 * w3[k] + e[k];
  *reinterpret_cast<f32x4*>(m + r * CM + c0) = v;
}

// Per-pair mask counts cnt[b][i][j] = sum_s mask[s,i] mask[s,j] (reference.py:645-646)
// from the k-major mask Mt [B][N][S'] (0/1 values, exact in fp32).  One workgroup per
// 32x32 tile, D[i][j]; its 4 waves take interleaved 64-sequence slices (16-byte operand
// loads straight from global, 4 k-steps in flight) and add their partial tiles in LDS.
__global__ __launch_bounds__(256) void opm_count_kernel(const op_t* __restrict__ Mt, float* __restrict__ cnt,
                                                        int B, int N, int Sp) {
  __shared__ f32x4 part[3][4][64];
  const int lane = threadIdx.x & 63, h = lane >> 5, mm = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nt = N / 32;
  const long t = blockIdx.x;
  const int tj = (int)(t % nt), ti = (int)((t / nt) % nt), b = (int)(t / ((long)nt * nt));
  const op_t* ra = Mt + ((long)b * N + 32 * ti + mm) * Sp + 8 * h;
  const op_t* rb = Mt + ((long)b * N + 32 * tj + mm) * Sp + 8 * h;
  f32x16 acc = zero16();
  for (int k0 = 64 * wid; k0 < Sp; k0 += 256) {
    opx8 fa[4], fb[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      fa[u] = ld_x8(ra + k0 + 16 * u);
      fb[u] = ld_x8(rb + k0 + 16 * u);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc = mfma32(fa[u], fb[u], acc);
  }
  if (wid > 0)
#pragma unroll
    for (int g = 0; g < 4; ++g) part[wid - 1][g][lane] = f32x4{acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]};
  __syncthreads();
  if (wid > 0) return;
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 p = part[w][g][lane];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[4 * g + e] += p[e];
    }
  float* out = cnt + ((long)b * N + 32 * ti) * N + 32 * tj + mm;
#pragma unroll
  for (int r = 0; r < 16; ++r) out[(long)acc_row(r, h) * N] = acc[r];
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
  opm_count_kernel<<<(unsigned)((long)B * (N / 32) * (N / 32)), 256, 0, st>>>(Mt, cnt, B, N, Sp);
  PF_CHECK_LAUNCH("opm_count_kernel");
  const long pairs = (long)B * N * N;
  opm_out_kernel<<<(unsigned)((pairs / 32 + 3) / 4), 256, 0, st>>>(Z, cnt, (const op_t*)a->w_o, a->b_o, a->z, B, N,
                                                                  X_LOAD_SCALE, a->accumulate);
  PF_CHECK_LAUNCH("opm_out_kernel");
  return PF_OK;
}

// Workspace of pf_pwa_fwd: logits [B*H][N][N] fp32, weights [B*H][N][N], v_t [B*H][32S][N],
// O [B*H][N][32S] (op_t).
extern "C" size_t pf_pwa_workspace_size(int B, int S, int N) {
  if (B <= 0 || S <= 0 || N <= 0) return 0;
  const size_t bh = (size_t)B * PH, nn = (size_t)N * N, sn = (size_t)S * PD * N;
  return bh * nn * sizeof(float) + (bh * nn + 2 * bh * sn) * sizeof(op_t);
}

extern "C" int pf_pwa_fwd(const pf_pwa_args* a) {
  if (!a) return pf_fail(PF_E_INVALID, "pf_pwa_fwd: null args");
  if (a->c_m != CM || a->C != CZ || a->H != PH || a->c_h != PD)
    return pf_fail(PF_E_INVALID, "pf_pwa_fwd: need c_m = 64, C = 128, 8 heads of 32 (got %d, %d, %d, %d)", a->c_m,
                   a->C, a->H, a->c_h);
  if (a->B <= 0 || a->S <= 0 || a->N <= 0 || a->N % 64)
    return pf_fail(PF_E_INVALID, "pf_pwa_fwd: need B, S > 0 and N a positive multiple of 64 (B=%d S=%d N=%d)", a->B,
                   a->S, a->N);
  if ((long)a->S * PD * a->N >= (1l << 31) || (long)a->B * a->N * a->N >= (1l << 31))
    return pf_fail(PF_E_INVALID, "pf_pwa_fwd: shape too large (B=%d S=%d N=%d)", a->B, a->S, a->N);
  if (!a->m || !a->out || !a->z || !a->norm_m_w || !a->norm_m_b || !a->norm_z_w || !a->norm_z_b || !a->w_m ||
      !a->w_g || !a->w_z || !a->w_o || !a->workspace)
    return pf_fail(PF_E_INVALID, "pf_pwa_fwd: null pointer argument");
  const size_t need = pf_pwa_workspace_size(a->B, a->S, a->N);
  if (a->workspace_bytes < need)
    return pf_fail(PF_E_INVALID, "pf_pwa_fwd: workspace too small (%zu < %zu bytes)", a->workspace_bytes, need);
  hipStream_t st = (hipStream_t)a->stream;
  const int B = a->B, S = a->S, N = a->N;
  const size_t bh = (size_t)B * PH, nn = (size_t)N * N, sn = (size_t)S * PD * N;
  float* logits = (float*)a->workspace;
  op_t* Wt = (op_t*)(logits + bh * nn);
  op_t* vt = Wt + bh * nn;
  op_t* O = vt + bh * sn;
  int rc = pf_pair_logits(a->z, a->norm_z_w, a->norm_z_b, a->w_z, logits, B, N, PH, a->eps, st);
  if (rc) return rc;
  pwa_softmax_kernel<<<(unsigned)((bh * N + 3) / 4), 256, 0, st>>>(logits, a->pair_mask, Wt, B, N);
  PF_CHECK_LAUNCH("pwa_softmax_kernel");
  const long vw = (long)B * S * (N / 32);
  pwa_proj_kernel<<<(unsigned)((vw + 7) / 8), 512, 0, st>>>(a->m, a->norm_m_w, a->norm_m_b, (const op_t*)a->w_m, vt,
                                                           B, S, N, a->eps);
  PF_CHECK_LAUNCH("pwa_proj_kernel");
  // rows (s, d) of v_t are the Nc dimension; S*32 is a multiple of 32
  if ((rc = pf_contract_rect(Wt, vt, O, 0, (int)bh, N, S * PD, N, 1.f, st))) return rc;
  const long ow = (long)B * N * ((S + 31) / 32);
  pwa_out_kernel<<<(unsigned)((ow + 7) / 8), 512, 0, st>>>(a->m, a->out, a->norm_m_w, a->norm_m_b,
                                                          (const op_t*)a->w_g, (const op_t*)a->w_o, O, B, S, N,
                                                          a->accumulate, a->eps);
  PF_CHECK_LAUNCH("pwa_out_kernel");
  return PF_OK;
}

extern "C" int pf_msa_embed(const int* msa, const float* has_deletion, const float* deletion_value,
                            const float* msa_paired, const float* s_emb, const float* w_t, float* m, int B, int S,
                            int N, int c_m, int n_tok, void* stream) {
  if (!msa || !s_emb || !w_t || !m) return pf_fail(PF_E_INVALID, "pf_msa_embed: null pointer");
  if (c_m != CM || B <= 0 || S <= 0 || N <= 0 || n_tok <= 0)
    return pf_fail(PF_E_INVALID, "pf_msa_embed: need c_m = 64 and positive B, S, N, n_tok (got %d %d %d %d %d)", c_m,
                   B, S, N, n_tok);
  const long rows = (long)B * S * N;
  const long threads = rows * (CM / 4);
  msa_embed_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      msa, has_deletion, deletion_value, msa_paired, s_emb, w_t, m, rows, S, N, n_tok);
  PF_CHECK_LAUNCH("msa_embed_kernel");
  return PF_OK;
}
