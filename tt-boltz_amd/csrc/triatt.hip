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
//              Q, K  op_t [B][N(row i)][H][N(j)][D]
//              Vt    op_t [B][N(row i)][H][D][N(k)]
//              bias2 fp32 [B][H][N(j)][N(k)]   (shared by all rows i)
//              M2    fp32 [B][N(i)][N(k)]      1e9*(mask-1)*log2(e), -inf for padding
//   ta_attn  flash attention.  A workgroup = 4 waves = 4 frame rows sharing one block of
//            64 queries, so every bias tile [64 q][64 k] is fetched once into LDS and
//            used by 4 rows; each wave loops over the 4 heads.  Scores are kept in the
//            transposed layout S^T[key][query]: each lane owns one query, the bias tile
//            is loaded straight into the MFMA accumulator, softmax statistics are per
//            lane (plus one cross-half exchange), and P feeds the P.V MFMA from
//            registers via the k-permutation of pf_common.h.  Online softmax with lazy
//            rescaling (the reference max only moves when it grows by > 2^8); row sums
//            come from v_dot2 over the rounded P that the MFMA consumes.  K/V and the
//            next bias tile are prefetched one step ahead.  Output O (normalized,
//            ungated) op_t [B][N(i)][N(j)][H*D].
//   ta_out   o-proj epilogue (persistent, W_g / W_o in LDS, output-aligned layout): gate
//            recomputed from LN(z) (MFMA), o*sigmoid(g) built in registers as linear_o's B
//            operand, residual added to the z values the lane loaded for the LayerNorm.
#include "pf_common.h"
#include "pf_internal.h"

namespace {

constexpr int C = 128, H = 4, D = 32, LDSW = 136;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float RESCALE_SLACK = 8.f;   // log2 units: P values stay <= 2^8 between rescales

typedef op_t opx2 __attribute__((ext_vector_type(2)));

PF_DEV float dot2_ones(const opx2& p, float acc) {
#ifdef PF_OPERAND_BF16
  const opx2 one = {(op_t)1.f, (op_t)1.f};
  return __builtin_amdgcn_fdot2_f32_bf16(p, one, acc, false);
#else
  const opx2 one = {(op_t)1.f, (op_t)1.f};
  return __builtin_amdgcn_fdot2(p, one, acc, false);
#endif
}

struct Blk32 { opx8 v[2]; };
// Load rows [0, nrows) of a [*][128] op_t block (rows >= nrows read as zero).
PF_DEV void blk32_load(const op_t* __restrict__ src, int nrows, int tid, Blk32& r) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int c = tid + 256 * q;
    const int row = c >> 4;
    r.v[q] = row < nrows ? ld_x8(src + row * C + (c & 15) * 8) : zero_x8();
  }
}
PF_DEV void blk32_store(op_t* lds, int tid, const Blk32& r) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int c = tid + 256 * q;
    st_x8(lds + (c >> 4) * LDSW + (c & 15) * 8, r.v[q]);
  }
}

// ---------------------------------------------------------------------------------
// Projection: one wave = 32 frame positions (ip, j0 .. j0+31).
// Weight blocks (32 rows each): 0-3 q heads, 4-7 k heads, 8-11 v heads, 12 bias.
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ta_proj_kernel(
    const float* __restrict__ z, const float* __restrict__ pair_mask,
    const float* __restrict__ lnw, const float* __restrict__ lnb,
    const op_t* __restrict__ wq, const op_t* __restrict__ wk, const op_t* __restrict__ wv,
    const op_t* __restrict__ wb, op_t* __restrict__ Q, op_t* __restrict__ K,
    op_t* __restrict__ Vt, float* __restrict__ bias2, float* __restrict__ M2,
    int B, int N, int n_valid, int ending, float qscale, float eps) {
  __shared__ __attribute__((aligned(16))) op_t lds[2][32 * LDSW];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, h = lane >> 5, m = lane & 31;
  const long NN = (long)N * N;
  const long pos0 = ((long)blockIdx.x * 4 + wid) * 32;
  const bool active = pos0 < (long)B * NN;

  int b = 0, ip = 0, j0 = 0;
  opx8 xf[8];
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
      // frame key j0+m of row ip: padding -> excluded; otherwise inf*(mask-1) (log2 units)
      const float mv = pair_mask ? pair_mask[pair] : 1.f;
      M2[((long)b * N + ip) * N + j0 + m] = j0 + m >= n_valid ? -INFINITY : 1e9f * (mv - 1.f) * LOG2E;
    }
  }

  auto src = [&](int bk) -> const op_t* {
    return bk < 4 ? wq + bk * 32 * C : bk < 8 ? wk + (bk - 4) * 32 * C
         : bk < 12 ? wv + (bk - 8) * 32 * C : wb;
  };
  Blk32 rw;
  blk32_load(src(0), 32, tid, rw);
  for (int bk = 0; bk < 13; ++bk) {
    op_t* lw = lds[bk & 1];
    blk32_store(lw, tid, rw);
    __syncthreads();
    if (bk + 1 < 13) blk32_load(src(bk + 1), bk + 1 < 12 ? 32 : H, tid, rw);
    if (!active) continue;
    f32x16 acc = zero16();
    if (bk < 8) {
      // normal orientation: rows = positions, cols = head dim
#pragma unroll
      for (int s = 0; s < 8; ++s) acc = mfma32(xf[s], ld_x8(lw + m * LDSW + 16 * s + 8 * h), acc);
      op_t* dst = bk < 4 ? Q : K;
      const float sc = bk < 4 ? qscale : 1.f;
      const long base = ((((long)b * N + ip) * H + (bk & 3)) * N + j0) * D;
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[base + acc_row(r, h) * D + m] = (op_t)(acc[r] * sc);
    } else {
      // transposed orientation: rows = head dim (or head for the bias), cols = positions
#pragma unroll
      for (int s = 0; s < 8; ++s) acc = mfma32(ld_x8(lw + m * LDSW + 16 * s + 8 * h), xf[s], acc);
      if (bk < 12) {
        const long base = (((long)b * N + ip) * H + (bk - 8)) * D * (long)N + j0 + m;
#pragma unroll
        for (int r = 0; r < 16; ++r) Vt[base + (long)acc_row(r, h) * N] = (op_t)acc[r];
      } else if (h == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) bias2[(((long)b * H + r) * N + ip) * N + j0 + m] = acc[r] * LOG2E;
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Flash attention.  OUT_F32 = false: O op_t [B][N][N][H*D] (frame pair layout);
// OUT_F32 = true: O fp32 [B][N][H][N][D] (the standalone attention-core API).
// ---------------------------------------------------------------------------------
constexpr int BP = 68;   // bias LDS pitch (floats): conflict-free b128 column reads

template <bool OUT_F32>
__global__ __launch_bounds__(256, 2) void ta_attn_kernel(
    const op_t* __restrict__ Q, const op_t* __restrict__ K, const op_t* __restrict__ Vt,
    const float* __restrict__ bias2, const float* __restrict__ M2, op_t* __restrict__ O16,
    float* __restrict__ O32, int N, int total) {
  __shared__ __attribute__((aligned(16))) float sBias[2][64 * BP];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, h = lane >> 5, m = lane & 31;
  const int nJB = N / 64, nIB = N / 4, nKB = N / 64;
  const int w = xcd_remap(blockIdx.x, total);
  const int b = w / (nIB * nJB);
  const int rem = w - b * nIB * nJB;
  const int ib = rem / nJB;
  const int j0 = (rem - ib * nJB) * 64;
  const int ip = ib * 4 + wid;          // this wave's frame row
  const long NN = (long)N * N;
  const float* Mr = M2 + ((long)b * N + ip) * N;

  // does any key of this row carry a mask/padding term?  (wave-uniform)
  bool masked = false;
  for (int k = lane; k < N; k += 64) masked |= (Mr[k] != 0.f);
  masked = __ballot(masked) != 0;

  const long rowbase = ((long)b * N + ip) * H;   // + head
  const int steps = H * nKB;

  // ---- prefetch state: bias tile (4 x float4 per thread), K and V fragments ----
  f32x4 breg[4];
  opx8 kreg[2][2], vreg[2][2];
  auto bias_load = [&](int t) {
    const int hd = t / nKB, kb0 = (t - hd * nKB) * 64;
    const float* src = bias2 + ((long)b * H + hd) * NN + (long)j0 * N + kb0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = tid + 256 * q;
      breg[q] = *reinterpret_cast<const f32x4*>(src + (long)(c >> 4) * N + (c & 15) * 4);
    }
  };
  auto kv_load = [&](int t) {
    const int hd = t / nKB, kb0 = (t - hd * nKB) * 64;
    const op_t* Kh = K + (rowbase + hd) * N * D;
    const op_t* Vh = Vt + (rowbase + hd) * D * N;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        kreg[kb][s] = ld_x8(Kh + (long)(kb0 + 32 * kb + m) * D + 16 * s + 8 * h);
        const op_t* vp = Vh + (long)m * N + kb0 + 32 * kb + 16 * s + 4 * h;
        vreg[kb][s] = cat44(ld_x4(vp), ld_x4(vp + 8));
      }
  };
  bias_load(0);
  kv_load(0);

  opx8 qf[2][2];
  f32x16 o[2];
  float mref[2], lsum[2];

  for (int t = 0; t < steps; ++t) {
    const int hd = t / nKB, kbi = t - hd * nKB, kb0 = kbi * 64;
    float* bt = sBias[t & 1];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = tid + 256 * q;
      *reinterpret_cast<f32x4*>(&bt[(c >> 4) * BP + (c & 15) * 4]) = breg[q];
    }
    opx8 kc[2][2], vc[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int s = 0; s < 2; ++s) { kc[kb][s] = kreg[kb][s]; vc[kb][s] = vreg[kb][s]; }
    __syncthreads();
    if (t + 1 < steps) { bias_load(t + 1); kv_load(t + 1); }

    if (kbi == 0) {   // head start
      const op_t* Qh = Q + (rowbase + hd) * N * D;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
#pragma unroll
        for (int s = 0; s < 2; ++s) qf[qb][s] = ld_x8(Qh + (long)(j0 + 32 * qb + m) * D + 16 * s + 8 * h);
        o[qb] = zero16();
        mref[qb] = -INFINITY;
        lsum[qb] = 0.f;
      }
    }

    // S^T = bias + K Q^T   (rows = keys, cols = queries)
    f32x16 sc[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 bv = *reinterpret_cast<const f32x4*>(&bt[(32 * qb + m) * BP + 32 * kb + 8 * g + 4 * h]);
          sc[kb][qb][4 * g + 0] = bv[0]; sc[kb][qb][4 * g + 1] = bv[1];
          sc[kb][qb][4 * g + 2] = bv[2]; sc[kb][qb][4 * g + 3] = bv[3];
        }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) sc[kb][qb] = mfma32(kc[kb][s], qf[qb][s], sc[kb][qb]);
    if (masked) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 mv = *reinterpret_cast<const f32x4*>(Mr + kb0 + 32 * kb + 8 * g + 4 * h);
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int e = 0; e < 4; ++e) sc[kb][qb][4 * g + e] += mv[e];
        }
    }

    opx8 pf[2][2][2];   // [qb][kb][ks]
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      float mx = sc[0][qb][0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sc[0][qb][r]);
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[1][qb][r]);
      mx = xor32_max(mx);
      if (__ballot(mx > mref[qb] + RESCALE_SLACK) != 0) {
        const float mnew = fmaxf(mref[qb], mx);
        const float alpha = exp2_fast(mref[qb] - mnew);
        mref[qb] = mnew;
        lsum[qb] *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) o[qb][r] *= alpha;
      }
      const float mr = mref[qb];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int t2 = 0; t2 < 8; t2 += 2) {
            opx2 pk;
            pk[0] = (op_t)exp2_fast(sc[kb][qb][8 * ks + t2] - mr);
            pk[1] = (op_t)exp2_fast(sc[kb][qb][8 * ks + t2 + 1] - mr);
            lsum[qb] = dot2_ones(pk, lsum[qb]);
            pf[qb][kb][ks][t2] = pk[0];
            pf[qb][kb][ks][t2 + 1] = pk[1];
          }
    }
    // O^T[d][q] += V^T[d][keys] * P^T[keys][q]  (keys in the accumulator's k-permutation)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) o[qb] = mfma32(vc[kb][ks], pf[qb][kb][ks], o[qb]);

    if (kbi == nKB - 1) {   // head end: normalize and store
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const float inv = rcp_fast(xor32_sum(lsum[qb]));
        const int j = j0 + 32 * qb + m;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          if (OUT_F32) {
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = o[qb][4 * g + e] * inv;
            *reinterpret_cast<f32x4*>(O32 + ((rowbase + hd) * N + j) * D + 8 * g + 4 * h) = v;
          } else {
            opx4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (op_t)(o[qb][4 * g + e] * inv);
            st_x4(O16 + (((long)b * N + ip) * N + j) * C + 32 * hd + 8 * g + 4 * h, v);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Output projection: z[pair(i, j)] (+)= linear_o(O[i, j] * sigmoid(linear_g(LN(z[pair])))).
// Persistent: one workgroup (8 waves) per CU keeps W_g and W_o in LDS; each wave walks
// tiles of 32 frame positions (ip, j0 .. j0+31).  Everything is in the output-aligned
// layout (pf_common.h): the gate comes out of D[channel][position] = W_g . LN(z) in the
// same channel order as the O values the lane loads, o * sigmoid(g) is directly the B
// operand of D[out][position] = W_o . (o * g), and the residual is the z the lane loaded.
// ---------------------------------------------------------------------------------
constexpr int TAO_WAVES = 8;
constexpr size_t TAO_LDS = (size_t)2 * C * LDSW * sizeof(op_t);

// resid: 0 -> out = update; 1 -> out = z_in + update (out may alias z_in); 2 -> out += update
__global__ __launch_bounds__(64 * TAO_WAVES, 1) void ta_out_kernel(
    const op_t* __restrict__ O, const float* z_in, float* out, const float* __restrict__ lnw,
    const float* __restrict__ lnb, const op_t* __restrict__ wg, const op_t* __restrict__ wo,
    int B, int N, int ending, int resid, float eps) {
  extern __shared__ __attribute__((aligned(16))) op_t tlds[];
  op_t* sWg = tlds;
  op_t* sWo = tlds + C * LDSW;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, h = lane >> 5, m = lane & 31;
  for (int c = tid; c < C * 16; c += 64 * TAO_WAVES) {
    const int row = c >> 4, col = (c & 15) * 8;
    st_x8(&sWg[row * LDSW + col], ld_x8(wg + row * C + col));
    st_x8(&sWo[row * LDSW + col], ld_x8(wo + row * C + col));
  }
  __syncthreads();
  const long NN = (long)N * N;
  const long ntiles = (long)B * NN / 32;
  for (long t = (long)blockIdx.x * TAO_WAVES + wid; t < ntiles; t += (long)gridDim.x * TAO_WAVES) {
    asm volatile("" ::: "memory");   // LayerNorm parameters are re-read, not pinned in VGPRs
    const long pos0 = t * 32;
    const int b = (int)(pos0 / NN);
    const long t0 = pos0 - (long)b * NN;
    const int ip = (int)(t0 / N);
    const int j = (int)(t0 - (long)ip * N) + m;
    const long zp = ending ? ((long)b * N + j) * N + ip : ((long)b * N + ip) * N + j;
    float zr[64];
    opx8 xf[8];
    load_row128_oa(z_in + zp * C, h, zr);
    ln128_oa_to_frag(zr, h, lnw, lnb, eps, xf);
    // o * sigmoid(g) as the B operand of the output projection (k order = output-aligned)
    opx8 og[8];
    const op_t* orow = O + (pos0 + m) * C;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const op_t* wrow = &sWg[(32 * cb + m) * LDSW];
      f32x16 g = zero16();
#pragma unroll
      for (int s = 0; s < 8; ++s) g = mfma32(wfrag_oa(wrow, s, h), xf[s], g);   // D[channel][position]
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
        const int q = 4 * cb + gg;            // chunk: channels oa_channel(q, h) + 0..3
        const opx4 ov = ld_x4(orow + oa_channel(q, h));
#pragma unroll
        for (int e = 0; e < 4; ++e)
          og[q >> 1][4 * (q & 1) + e] = (op_t)((float)ov[e] * sigmoidf_fast(g[4 * gg + e]));
      }
    }
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) {
      const op_t* wrow = &sWo[(32 * ob + m) * LDSW];
      f32x16 acc = zero16();
#pragma unroll
      for (int s = 0; s < 8; ++s) acc = mfma32(wfrag_oa(wrow, s, h), og[s], acc);   // D[out][position]
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
        const int q = 4 * ob + gg;
        float* dst = out + zp * C + oa_channel(q, h);
        f32x4 v;
        if (resid == 2) v = *reinterpret_cast<const f32x4*>(dst);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float u = acc[4 * gg + e];
          v[e] = resid == 1 ? zr[4 * q + e] + u : resid == 2 ? v[e] + u : u;
        }
        *reinterpret_cast<f32x4*>(dst) = v;
      }
    }
  }
}

// Layout conversion for the standalone attention core (fp32 API tensors -> kernel layout).
__global__ void ta_prep_qkv_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                   const float* __restrict__ v, float qs, op_t* __restrict__ Q,
                                   op_t* __restrict__ K, op_t* __restrict__ Vt, long rows, int N) {
  // rows = B*N*H sequences of N x D; element e of sequence r: (j, d) = (e / D, e % D)
  const long total = rows * N * D;
  for (long e = (long)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (long)gridDim.x * blockDim.x) {
    const long r = e / ((long)N * D);
    const int jd = (int)(e - r * N * D);
    const int j = jd / D, d = jd - j * D;
    Q[e] = (op_t)(q[e] * qs);
    K[e] = (op_t)k[e];
    Vt[r * N * D + (long)d * N + j] = (op_t)v[e];
  }
}

__global__ void ta_prep_bias_kernel(const float* __restrict__ bias, const float* __restrict__ mask,
                                    float* __restrict__ bias2, float* __restrict__ M2,
                                    long nbias, long nmask, int N, int n_valid) {
  for (long e = (long)blockIdx.x * blockDim.x + threadIdx.x; e < nbias; e += (long)gridDim.x * blockDim.x) {
    bias2[e] = bias[e] * LOG2E;
    if (e < nmask) {
      const int key = (int)(e % N);
      M2[e] = key >= n_valid ? -INFINITY : mask ? 1e9f * (mask[e] - 1.f) * LOG2E : 0.f;
    }
  }
}

struct TaBuffers {
  op_t *Q, *K, *Vt, *O;
  float *bias2, *M2;
};

size_t ta_buffers_size(int B, int N) {
  const size_t e = (size_t)B * N * H * N * D;
  return 4 * e * sizeof(op_t) + ((size_t)B * H * N * N + (size_t)B * N * N) * sizeof(float);
}

TaBuffers ta_buffers(void* ws, int B, int N) {
  const size_t e = (size_t)B * N * H * N * D;
  TaBuffers t;
  t.Q = (op_t*)ws;
  t.K = t.Q + e;
  t.Vt = t.K + e;
  t.O = t.Vt + e;
  t.bias2 = (float*)(t.O + e);
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
  if (a->n_valid < 0 || a->n_valid > a->N)
    return pf_fail(PF_E_INVALID, "pf_triatt_fwd: n_valid %d outside [0, N=%d]", a->n_valid, a->N);
  hipStream_t st = (hipStream_t)a->stream;
  const int B = a->B, N = a->N;
  const int n_valid = a->n_valid ? a->n_valid : N;
  TaBuffers t = ta_buffers(a->workspace, B, N);
  const float qscale = LOG2E / sqrtf((float)D);
  const long positions = (long)B * N * N;
  const int grid_pos = (int)((positions / 32 + 3) / 4);
  ta_proj_kernel<<<grid_pos, 256, 0, st>>>(a->z_in, a->pair_mask, a->ln_w, a->ln_b,
                                           (const op_t*)a->w_q, (const op_t*)a->w_k, (const op_t*)a->w_v,
                                           (const op_t*)a->w_bias, t.Q, t.K, t.Vt, t.bias2, t.M2, B, N,
                                           n_valid, a->ending, qscale, a->eps);
  PF_CHECK_LAUNCH("ta_proj_kernel");
  const int total = B * (N / 4) * (N / 64);
  ta_attn_kernel<false><<<total, 256, 0, st>>>(t.Q, t.K, t.Vt, t.bias2, t.M2, t.O, nullptr, N, total);
  PF_CHECK_LAUNCH("ta_attn_kernel");
  {
    static bool attr = false;
    if (!attr) {
      if (hipFuncSetAttribute((const void*)ta_out_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)TAO_LDS) != hipSuccess)
        return pf_fail(PF_E_LAUNCH, "ta_out_kernel: cannot reserve %zu bytes of LDS", TAO_LDS);
      attr = true;
    }
    const int grid = (int)min((long)device_cus(), (positions / 32 + TAO_WAVES - 1) / TAO_WAVES);
    const int resid = !a->accumulate ? 0 : (a->out == a->z_in ? 1 : 2);
    ta_out_kernel<<<grid, 64 * TAO_WAVES, TAO_LDS, st>>>(t.O, a->z_in, a->out, a->ln_w, a->ln_b,
                                                         (const op_t*)a->w_g, (const op_t*)a->w_o, B, N, a->ending,
                                                         resid, a->eps);
  }
  PF_CHECK_LAUNCH("ta_out_kernel");
  return PF_OK;
}

extern "C" size_t pf_tri_attention_workspace_size(int B, int N, int H_, int D_) {
  if (B <= 0 || N <= 0 || H_ != H || D_ != D) return 0;
  return ta_buffers_size(B, N);
}

extern "C" int pf_tri_attention(const float* q, const float* k, const float* v, const float* bias,
                                const float* mask, float scale, float* o, int B, int N, int H_, int D_,
                                int n_valid, void* workspace, size_t workspace_bytes, void* stream) {
  if (H_ != H || D_ != D)
    return pf_fail(PF_E_INVALID, "pf_tri_attention: only H=4, D=32 supported (got H=%d D=%d)", H_, D_);
  if (B <= 0 || N <= 0 || N % 64)
    return pf_fail(PF_E_INVALID, "pf_tri_attention: need B > 0 and N a positive multiple of 64 (B=%d N=%d)", B, N);
  if (n_valid < 0 || n_valid > N)
    return pf_fail(PF_E_INVALID, "pf_tri_attention: n_valid %d outside [0, N=%d]", n_valid, N);
  if (n_valid == 0) n_valid = N;
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
  ta_prep_bias_kernel<<<1024, 256, 0, st>>>(bias, mask, t.bias2, t.M2, (long)B * H * N * N, (long)B * N * N, N,
                                            n_valid);
  PF_CHECK_LAUNCH("ta_prep_bias_kernel");
  const int total = B * (N / 4) * (N / 64);
  ta_attn_kernel<true><<<total, 256, 0, st>>>(t.Q, t.K, t.Vt, t.bias2, t.M2, nullptr, o, N, total);
  PF_CHECK_LAUNCH("ta_attn_kernel");
  return PF_OK;
}
