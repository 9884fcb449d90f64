// Triangle multiplication (outgoing / incoming) for gfx950.
//
// Replaces TriangleMultiplication{Outgoing,Incoming}.forward
// (tt_bio/reference.py:387-561) and the ttnn TriangleMultiplication
// (tt_bio/tenstorrent.py:351-503).  Three launches per call:
//
//   tm_proj     LN_in(z) -> [p_in | g_in] projection (MFMA) -> a = p*sigmoid(g)*mask,
//               written as channel-major operand planes opA/opB [B][128][N][N] (op_t).
//               The plane layout already folds the direction: for both directions
//               the contraction below is  X[c][i][j] = sum_k opA[c][i][k] * opB[c][j][k].
//                 outgoing: opA[c][i][k] = a[i,k,c],  opB[c][j][k] = b[j,k,c]
//                 incoming: opA[c][i][k] = a[k,i,c],  opB[c][j][k] = b[k,j,c]
//   tm_contract 128 (x B) independent N x N x N GEMMs, fp32 accumulate, XCD-aware tile
//               order.  X is stored as op_t (half the traffic of fp32) times a per-call
//               power of two chosen from max |a|, |b| (x_store_scale in pf_common.h), so
//               fp16 neither overflows nor drops into subnormals for any weight scale.
//   tm_out      LN_out(X) -> p_out, LN_in(z) -> g_out (recomputed, so no gate tensor
//               goes through HBM), update = p * sigmoid(g), residual into z.
#include "pf_common.h"
#include "pf_internal.h"

namespace {

constexpr int C = 128;        // c_z
constexpr float LOG2E = 1.4426950408889634f;
constexpr int LDSW = 136;     // padded LDS row stride (elements) for [rows][128] tiles

// A [32][128] op_t block moved by 256 threads: 512 chunks of 16 B, 2 per thread.
struct Blk32 { opx8 v[2]; };
PF_DEV void blk32_load(const op_t* __restrict__ src, int tid, Blk32& r) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int c = tid + 256 * q;
    r.v[q] = ld_x8(src + (c >> 4) * C + (c & 15) * 8);
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
// Input projection.  Persistent: one workgroup (8 waves, two per SIMD) per CU keeps p_in and
// g_in ([2 CC][CC] each, op_t as given, so rounded once) resident in LDS, with the LayerNorm's
// beta folded into fp32 offsets W beta added in the epilogue (gamma scales the normalized z
// before its rounding to op_t).  Every wave walks tiles of 32
// consecutive positions of one operand-plane row (orow, ocol0 .. ocol0+31) and loads the next
// tile's z rows while it computes the current one.  The projection is formed as
// D[position][channel]; each 32x32 output block goes through a per-wave LDS stage so that it
// leaves as 16-byte stores, four lanes per 64-byte plane-row segment (a full segment per
// instruction writes faster than register-permuted 32-byte halves).  The channel-block loop is
// unrolled, so the number of stores issued after the prefetch is static, with a scheduling
// barrier per block to keep each block's LDS reads and MFMAs inside its own iteration.
// ---------------------------------------------------------------------------------
constexpr int TMP_WAVES = 8;
constexpr int SPITCH = 40;     // output staging pitch (elements): one 32-position row + 16 B
template <int CC>
constexpr int tmp_waves() { return TMP_WAVES; }
// CC = c_z (64 or 128).  LDS: gamma [CC] and the offsets W_p beta [2 CC], -log2(e) W_g beta
// [2 CC] (fp32, first: small immediate offsets), then W_p, W_g [2 CC][CC + 8] op_t, the per-wave
// output stages and the per-wave maxima.
template <int CC>
constexpr size_t tmp_lds() {
  return 5 * CC * sizeof(float) + (size_t)2 * 2 * CC * (CC + 8) * sizeof(op_t) +
         (size_t)TMP_WAVES * 32 * SPITCH * sizeof(op_t) + TMP_WAVES * sizeof(float);
}

// offb (optional, fp32 [4 CC]): the exact W_p beta, W_g beta (else computed from the op_t
// weights); with p_lo / g_lo (the weights' residuals) and the stats partials also the mean
// correction (see pair_stats_kernel).
template <int CC, bool MASK>
__global__ __launch_bounds__(64 * TMP_WAVES, 1) void tm_proj_kernel(
    const float* __restrict__ z, const float* __restrict__ mask,
    const float* __restrict__ lnw, const float* __restrict__ lnb,
    const op_t* __restrict__ w_p, const op_t* __restrict__ w_g,
    op_t* __restrict__ opA, op_t* __restrict__ opB, float* __restrict__ amax_parts, int B, int N, int incoming,
    float eps, const float* __restrict__ offb, const op_t* __restrict__ p_lo, const op_t* __restrict__ g_lo,
    const float* __restrict__ stats) {
  constexpr int LW = CC + 8, KS = CC / 16;
  extern __shared__ __attribute__((aligned(16))) op_t wlds[];
  float* gam = reinterpret_cast<float*>(wlds);
  float* cbias = gam + CC;   // [0, 2 CC): W_p beta, [2 CC, 4 CC): -log2(e) W_g beta
  op_t* lp = wlds + 5 * CC * 2;
  op_t* lg = lp + 2 * CC * LW;
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, m = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  op_t* stg = lg + 2 * CC * LW + wid * 32 * SPITCH;
  float* wave_amax = reinterpret_cast<float*>(lg + 2 * CC * LW + TMP_WAVES * 32 * SPITCH);
  float* mu = reinterpret_cast<float*>(lg + 2 * CC * LW);   // the output stages, free until the tile loop
  constexpr int NT = 64 * TMP_WAVES;
  static_assert(4 * CC <= NT, "one offset row per thread");
  const int orow = tid;   // this thread's offset row (W beta): 0 .. 4 CC - 1
  opx8 rv[CC / 8];        // the row behind it: the residual (mean correction) or the weight
  float offb_v = 0.f;
  // set-up in two batches of global loads (each issued whole before its first use): the weights
  // and partials, then, while the statistics reduce, the residual rows of the mean correction
  const bool meanfix = offb && stats;
  {
    opx8 vp[stage_per<NT, 2 * CC, CC>()], vg[stage_per<NT, 2 * CC, CC>()];
    stage_load<NT, 2 * CC, CC>(w_p, vp);
    stage_load<NT, 2 * CC, CC>(w_g, vg);
    const float gv = tid < CC ? lnw[tid] : 0.f;
    float pv[stats_per<NT>()];
    if (meanfix) stats_load<NT>(stats, pv);
    if (offb && orow < 4 * CC) offb_v = offb[orow];
    stage_store<NT, 2 * CC, CC>(lp, LW, vp);
    stage_store<NT, 2 * CC, CC>(lg, LW, vg);
    if (tid < CC) gam[tid] = gv;
    if constexpr (CC == C)
      if (meanfix && orow < 4 * CC) {
        const op_t* lo = orow < 2 * CC ? p_lo + orow * CC : g_lo + (orow - 2 * CC) * CC;
#pragma unroll
        for (int c = 0; c < CC / 8; ++c) rv[c] = ld_x8(lo + 8 * c);
      }
    if (meanfix) stats_reduce<NT>(pv, mu, mu + PS_C);
  }
  __syncthreads();
  if (orow < 4 * CC) {   // offsets W beta (one row per thread)
    float acc = 0.f;
    if (offb) {
      if constexpr (CC == C) acc = corrected_offset_regs<true>(offb_v, rv, stats != nullptr, gam, mu);
    } else {   // from the staged weights (rows 16-byte aligned)
      const op_t* w = orow < 2 * CC ? lp + orow * LW : lg + (orow - 2 * CC) * LW;
#pragma unroll
      for (int c = 0; c < CC / 8; ++c) {
        const opx8 w8 = ld_x8(w + 8 * c);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += (float)w8[e] * lnb[8 * c + e];
      }
    }
    cbias[orow] = orow < 2 * CC ? acc : -LOG2E * acc;
  }
  __syncthreads();
  const uint32_t ntiles = (uint32_t)B * N * N / 32;
  const uint32_t stride = gridDim.x * TMP_WAVES;
  auto tile_pair = [&](uint32_t t, int& b, int& orow, int& ocol0) PF_INLINE -> long {
    const PosTile pt = pos_tile(t, N);
    b = pt.b;
    orow = pt.r;
    ocol0 = pt.c0;
    const int zi = incoming ? ocol0 + m : orow;
    const int zj = incoming ? orow : ocol0 + m;
    return ((long)b * N + zi) * N + zj;
  };
  float amax = 0.f;   // max |a|, |b| before rounding (rounding is monotonic: round it once at the end)
  float x[CC / 2];    // this tile's z rows, then the next tile's (in flight during the MFMAs)
  float maskn = 1.f;
  uint32_t t = blockIdx.x * TMP_WAVES + wid;
  if (t < ntiles) {
    int b_, r_, c_;
    const long pair = tile_pair(t, b_, r_, c_);
    load_row_frag<CC>(z + pair * CC, h, x);
    if (MASK) maskn = mask[pair];
  }
  for (; t < ntiles; t += stride) {
    int cb_b, cb_orow, cb_ocol0;
    tile_pair(t, cb_b, cb_orow, cb_ocol0);
    opx8 xf[KS];
    const float maskv = maskn;
    ln_gamma_to_frag<CC>(x, h, gam, eps, xf);
    float mr[16];
    if (MASK) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mr[r] = __shfl(maskv, acc_row(r, h));
    }
    if (t + stride < ntiles) {
      int b_, r_, c_;
      const long pn = tile_pair(t + stride, b_, r_, c_);
      load_row_frag<CC>(z + pn * CC, h, x);
      if (MASK) maskn = mask[pn];
    }
    // software pipeline: the MFMAs of block cb + 1 are issued before block cb's epilogue
    f32x16 apq[2], agq[2];
    auto mm = [&](int cb, f32x16& ap, f32x16& ag) PF_INLINE {
      const op_t* wp = lp + (32 * cb + m) * LW + 8 * h;
      const op_t* wg = lg + (32 * cb + m) * LW + 8 * h;
      ap = zero16();
      ag = zero16();
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        ap = mfma32(xf[s], ld_x8(wp + 16 * s), ap);   // rows = position, cols = output channel
        ag = mfma32(xf[s], ld_x8(wg + 16 * s), ag);
      }
    };
    mm(0, apq[0], agq[0]);
#pragma unroll
    for (int cb = 0; cb < 2 * CC / 32; ++cb) {
      __builtin_amdgcn_sched_barrier(0);
      if (cb + 1 < 2 * CC / 32) mm(cb + 1, apq[(cb + 1) & 1], agq[(cb + 1) & 1]);
      const float cp = cbias[32 * cb + m], cg = cbias[2 * CC + 32 * cb + m];
      const f32x16& ap = apq[cb & 1];
      const f32x16& ag = agq[cb & 1];
      // lane (channel m, half h) holds positions 8g + 4h + e: stage [channel][position]
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        opx4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g + e;
          float u = (ap[r] + cp) * rcp_fast(1.f + exp2_fast(fmaf(ag[r], -LOG2E, cg)));
          if (MASK) u *= mr[r];
          amax = fmaxf(amax, fabsf(u));
          v[e] = (op_t)u;
        }
        st_x4(stg + m * SPITCH + 8 * g + 4 * h, v);
      }
      op_t* dst = (cb < CC / 32 ? opA : opB) + (((long)cb_b * CC + 32 * (cb % (CC / 32))) * N + cb_orow) * N + cb_ocol0;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int row = 16 * q + (lane >> 2), chunk = lane & 3;
        st_x8(dst + (long)row * N * N + 8 * chunk, ld_x8(stg + row * SPITCH + 8 * chunk));
      }
    }
  }
  // the workgroup's max |a|, |b| as stored -> amax_parts[blockIdx.x] (the contraction's scale input)
  amax = fabsf((float)(op_t)wave_max(amax));
  if (lane == 0) wave_amax[wid] = amax;
  __syncthreads();
  if (tid == 0) {
    float mx = wave_amax[0];
#pragma unroll
    for (int w = 1; w < TMP_WAVES; ++w) mx = fmaxf(mx, wave_amax[w]);
    amax_parts[blockIdx.x] = mx;
  }
}

// ---------------------------------------------------------------------------------
// Batched contraction X[p][i][j] = sum_k A[p][i][k] * B[p][j][k] over planes p.
// ---------------------------------------------------------------------------------
constexpr int BM = 128, BN = 128, BK = 64, LDK = BK + 8;

// The output is scaled by out_scale, or, when nparts > 0, by x_store_scale of the operand
// maxima in amax_parts (K = the contraction length).
template <typename OutT>
__global__ __launch_bounds__(256) void tm_contract_kernel(
    const op_t* __restrict__ A, const op_t* __restrict__ Bop, OutT* __restrict__ X,
    int N, int tpd, int total, float out_scale, const float* __restrict__ amax_parts, int nparts) {
  __shared__ __attribute__((aligned(16))) op_t sA[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) op_t sB[2][BN * LDK];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, h = lane >> 5, m = lane & 31;
  const int wm = wid >> 1, wn = wid & 1;
  const int w = xcd_remap(blockIdx.x, total);
  const int tiles = tpd * tpd;
  const long plane = w / tiles;
  const int t = w - (int)plane * tiles;
  const int i0 = (t / tpd) * BM, j0 = (t % tpd) * BN;
  const long NN = (long)N * N;
  const op_t* Ap = A + plane * NN;
  const op_t* Bp = Bop + plane * NN;

  // global -> register staging: rows (tid >> 3) + 32*q, 16-byte chunk (tid & 7)
  const int lrow = tid >> 3, lcol = (tid & 7) * 8;
  const op_t* ga[4];
  const op_t* gb[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int ra = min(i0 + lrow + 32 * q, N - 1);
    const int rb = min(j0 + lrow + 32 * q, N - 1);
    ga[q] = Ap + (long)ra * N + lcol;
    gb[q] = Bp + (long)rb * N + lcol;
  }
  opx8 ra_[4], rb_[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) { ra_[q] = ld_x8(ga[q]); rb_[q] = ld_x8(gb[q]); }

  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c) acc[a][c] = zero16();

  const int nk = N / BK;
  for (int kt = 0; kt < nk; ++kt) {
    op_t* la = sA[kt & 1];
    op_t* lb = sB[kt & 1];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      st_x8(la + (lrow + 32 * q) * LDK + lcol, ra_[q]);
      st_x8(lb + (lrow + 32 * q) * LDK + lcol, rb_[q]);
    }
    __syncthreads();
    if (kt + 1 < nk) {
      const int ko = (kt + 1) * BK;
#pragma unroll
      for (int q = 0; q < 4; ++q) { ra_[q] = ld_x8(ga[q] + ko); rb_[q] = ld_x8(gb[q] + ko); }
    }
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      opx8 fa[2], fb[2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        fa[x] = ld_x8(la + (wm * 64 + 32 * x + m) * LDK + 16 * s + 8 * h);
        fb[x] = ld_x8(lb + (wn * 64 + 32 * x + m) * LDK + 16 * s + 8 * h);
      }
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc[a][c] = mfma32(fa[a], fb[c], acc[a][c]);
    }
  }

  if (nparts > 0) out_scale = x_store_scale(planes_amax(amax_parts, nparts), N);
  OutT* Xp = X + plane * NN;
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int j = j0 + wn * 64 + 32 * c + m;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = i0 + wm * 64 + 32 * a + acc_row(r, h);
        if (i < N && j < N) Xp[(long)i * N + j] = (OutT)(acc[a][c][r] * out_scale);
      }
    }
}

// Large-N contraction: a 256x256 output tile per workgroup of 8 waves (two per SIMD) in
// 2 (i) x 4 (j); each wave owns 128 (i) x 64 (j) = 4x2 MFMA 32x32 tiles (128 fp32
// accumulators per lane), so while one wave of a SIMD waits on LDS reads or the slab
// barrier the other issues MFMAs (measured 5-10 % faster than 4 waves of 128x128 on every
// shape used here).  The wave computes the transposed tile D[j][i] = sum_k B[j][k] A[i][k],
// so a lane's accumulator registers 4g..4g+3 hold 4 consecutive j of one i and the
// epilogue writes 16-byte runs.
//
// Operands move global -> LDS with global_load_lds_dwordx4 (lane l of an instruction
// lands at LDS base + 16*l), so no VGPRs are spent on staging, through a 2-deep ring of
// [256][64] slabs per operand: every DMA request is a whole 128-byte row segment, and
// slab kt+1 is in flight while slab kt is consumed.  Within a slab the fragment reads of
// the next k-step are interleaved one per MFMA of the current one.  One workgroup fills a CU,
// so when the tile count leaves a last round on half of the CUs or fewer (N = 768: 1152 tiles
// on 256 CUs), those tiles are split in two 128-row halves and the round takes half as long.
// ---------------------------------------------------------------------------------
constexpr int BM2 = 256;
constexpr int TMD_WAVES = 8;


// Slab layout: chunk c (0..7, 16 bytes) of row r at position 8r + (c ^ swz8(r)) with
// swz8(r) = ((r>>1)&7) ^ ((r&1)<<2).  A fragment read takes one chunk from each of 32
// consecutive rows; for any 8 (or 16) consecutive aligned rows the positions fall in 8
// (16) distinct 16-byte bank groups, so reads are conflict-free whether the LDS serves
// 8 or 16 lanes of a 128-bit read per cycle.
PF_DEV int slab_swz8(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }
constexpr int DK8 = 64;
constexpr int DSLAB8 = BM2 * DK8;
constexpr size_t TMD8_LDS_BYTES = (size_t)2 * 2 * DSLAB8 * sizeof(op_t);

// One output tile of 64 XN (i) x 256 (j): XN = 4 is the whole 256x256 tile; XN = 2 is half of
// one (rows i0 .. i0 + 127), used for the tiles of a last, partial round of the chip (below).
// A half tile's waves own 64 (i) x 64 (j) each and read 4 fragments per 4 MFMAs.
template <int XN, typename OutT>
PF_DEV void contract_tile(const op_t* __restrict__ A, const op_t* __restrict__ Bop, OutT* __restrict__ X, int M,
                          int Nc, int K, long plane, int i0, int j0, float out_scale,
                          const float* __restrict__ amax_parts, int nparts, op_t* smem) {
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, m = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid >> 2, wn = wid & 3;
  constexpr int QA = XN;   // A-slab DMA instructions per wave (64 XN rows over 8 waves)

  // DMA: instruction q of this wave covers slab rows (QA*wid + q)*8 (A; 4*wid + q for B) + (lane >> 3)
  int offA[QA], offB[4];
#pragma unroll
  for (int q = 0; q < QA; ++q) {
    const int r = (QA * wid + q) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ slab_swz8(r);
    offA[q] = min(i0 + r, M - 1) * K + 8 * c;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (4 * wid + q) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ slab_swz8(r);
    offB[q] = min(j0 + r, Nc - 1) * K + 8 * c;
  }
  const op_t* Ap = A + plane * M * K;
  const op_t* Bp = Bop + plane * Nc * K;
  auto issue = [&](int kt) {
    op_t* sa = smem + (kt & 1) * 2 * DSLAB8;
    op_t* sb = sa + DSLAB8;
    const int ko = kt * DK8;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q < QA) __builtin_amdgcn_global_load_lds(Ap + offA[q] + ko, sa + (QA * wid + q) * 512, 16, 0, 0);
      __builtin_amdgcn_global_load_lds(Bp + offB[q] + ko, sb + (4 * wid + q) * 512, 16, 0, 0);
    }
  };
  const int swz = slab_swz8(m);   // rows base + 32x + m: bits 0-3 of the row are those of m
  const int rdA = (wm * 32 * XN + m) * DK8, rdB = (wn * 64 + m) * DK8;
  auto read_frags = [&](int kt, int s, opx8 (&fa)[XN], opx8 (&fb)[2]) {
    const op_t* sa = smem + (kt & 1) * 2 * DSLAB8;
    const op_t* sb = sa + DSLAB8;
    const int cs = 8 * ((2 * s + h) ^ swz);
#pragma unroll
    for (int x = 0; x < XN; ++x) fa[x] = ld_x8(sa + rdA + 32 * x * DK8 + cs);
#pragma unroll
    for (int y = 0; y < 2; ++y) fb[y] = ld_x8(sb + rdB + 32 * y * DK8 + cs);
  };
  f32x16 acc[2][XN];
#pragma unroll
  for (int y = 0; y < 2; ++y)
#pragma unroll
    for (int x = 0; x < XN; ++x) acc[y][x] = zero16();
  auto mma = [&](const opx8 (&fa)[XN], const opx8 (&fb)[2]) {
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int x = 0; x < XN; ++x) acc[y][x] = mfma32(fb[y], fa[x], acc[y][x]);
  };
  // the XN + 2 fragment reads of the next k-step, one after each of the first XN + 2 MFMAs
  auto interleave = [&]() {
#pragma unroll
    for (int q = 0; q < XN + 2; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if constexpr (2 * XN > XN + 2) __builtin_amdgcn_sched_group_barrier(0x008, XN - 2, 0);
  };

  const int nk = K / DK8;
  issue(0);
  opx8 f0a[XN], f0b[2], f1a[XN], f1b[2];
  for (int kt = 0; kt < nk; ++kt) {
    // slab kt landed (slab kt+1 not yet issued); the barrier also tells every wave that
    // slab kt-1's buffer is free, so slab kt+1 can go into it
    __builtin_amdgcn_s_waitcnt(vmcnt_le(0));
    __builtin_amdgcn_s_barrier();
    if (kt + 1 < nk) issue(kt + 1);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(kt, 0, f0a, f0b);
    read_frags(kt, 1, f1a, f1b);
    mma(f0a, f0b);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(kt, 2, f0a, f0b);
    mma(f1a, f1b);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    read_frags(kt, 3, f1a, f1b);
    mma(f0a, f0b);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    mma(f1a, f1b);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (nparts > 0) out_scale = x_store_scale(planes_amax(amax_parts, nparts), K);
  OutT* Xp = X + plane * M * Nc;
#pragma unroll
  for (int x = 0; x < XN; ++x) {
    const int ib = i0 + wm * 32 * XN + 32 * x;
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int jb = j0 + wn * 64 + 32 * y;
      if (ib >= M || jb >= Nc) continue;
      if constexpr (sizeof(OutT) == 4) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          f32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[y][x][4 * g + e] * out_scale;
          *reinterpret_cast<f32x4*>(Xp + (long)(ib + m) * Nc + jb + 8 * g + 4 * h) = v;
        }
      } else {
        store_runs16((op_t*)(Xp + (long)(ib + m) * Nc + jb), acc[y][x], out_scale, h);   // 16-byte runs
      }
    }
  }
}

// Workgroups 0 .. full-1 take whole tiles 0 .. full-1; the `ntiles - full` tiles after them
// (a last round that would leave at least half of the CUs idle) go to two workgroups each, one
// per 128-row half, so that round takes about half as long.  Both ranges are mapped XCD-aware
// on their own, so the workgroups of one plane share an XCD's L2.
template <typename OutT>
__global__ __launch_bounds__(64 * TMD_WAVES, 1) void tm_contract_dma_kernel(
    const op_t* __restrict__ A, const op_t* __restrict__ Bop, OutT* __restrict__ X,
    int M, int Nc, int K, int tn, int ntiles, int full, float out_scale, const float* __restrict__ amax_parts,
    int nparts) {
  extern __shared__ __attribute__((aligned(16))) op_t smem[];
  const int tiles = ((M + BM2 - 1) / BM2) * tn;   // per plane
  const int bid = blockIdx.x;
  if (bid < full) {
    const int w = xcd_remap(bid, full);
    const long plane = w / tiles;
    const int t = w - (int)plane * tiles;
    contract_tile<4, OutT>(A, Bop, X, M, Nc, K, plane, (t / tn) * BM2, (t % tn) * BM2, out_scale, amax_parts,
                           nparts, smem);
  } else {
    const int hw = xcd_remap(bid - full, 2 * (ntiles - full));
    const int w = full + (hw >> 1);
    const long plane = w / tiles;
    const int t = w - (int)plane * tiles;
    contract_tile<2, OutT>(A, Bop, X, M, Nc, K, plane, (t / tn) * BM2 + (hw & 1) * (BM2 / 2), (t % tn) * BM2,
                           out_scale, amax_parts, nparts, smem);
  }
}

// ---------------------------------------------------------------------------------
// Output: z[i,j,:] (+)= p_out(LN_out(X[:,i,j])) * sigmoid(g_out(LN_in(z[i,j,:]))).
// Persistent: one workgroup (8 waves) per CU keeps p_out / g_out in LDS (op_t as given, so
// rounded once) with both LayerNorms' beta folded into fp32 offsets W beta, added to the
// products (gamma scales the normalized values before their rounding to op_t); each wave walks
// tiles of 32 consecutive pairs.  The tile's X slice (CC channels x 32 pairs, 64-byte rows of
// the planes) comes in with 16-byte loads into a per-wave LDS stage and is read back per
// channel.  Both products are formed as D[channel][pair] in the output-aligned layout, so the
// residual z values the wave loaded for LN_in are the ones it adds to (no second read of z).
// Weight rows are CC + 4 op_t apart, so the 8-byte fragment reads of 32 rows fall on distinct
// banks.
// ---------------------------------------------------------------------------------
constexpr int TMO_WAVES = 8, XSP = 40;   // per-wave X stage: [CC channels][32 pairs + 8]
// LDS: the offsets W_p beta_out [CC], -log2(e) W_g beta_in [CC] and gamma_out [CC], gamma_in [CC]
// (fp32, first: small immediate offsets), then W_p, W_g [CC][CC + 4] op_t, (HILO) W_p's residual
// in the same layout, then the per-wave X stages (HILO: half the channels, filled twice a tile)
template <int CC, bool HILO = false>
constexpr size_t tmo_lds() {
  return 4 * CC * sizeof(float) + (size_t)(HILO ? 3 : 2) * CC * (CC + 4) * sizeof(op_t) +
         (size_t)TMO_WAVES * (HILO ? CC / 2 : CC) * XSP * sizeof(op_t);
}

// resid: 0 -> out = update; 1 -> out = z_in + update (out may alias z_in); 2 -> out += update
// X is read back times x_scale, or, when nparts > 0, divided by the contraction's
// x_store_scale of the operand maxima in amax_parts (contraction length N).
// HILO: p_out comes with its rounding residual w_pout_lo = p_out - p_out16 (op_t) and the
// output projection runs on both (two MFMAs per fragment: weights good to ~2^-22 of their size).
template <typename XT, int CC, bool HILO = false>
__global__ __launch_bounds__(64 * TMO_WAVES, 1) void tm_out_kernel(
    const XT* __restrict__ X, float x_scale, const float* __restrict__ amax_parts, int nparts,
    const float* z_in, float* out,
    const float* __restrict__ lni_w, const float* __restrict__ lni_b,
    const float* __restrict__ lno_w, const float* __restrict__ lno_b,
    const op_t* __restrict__ w_pout, const op_t* __restrict__ w_gout, const op_t* __restrict__ w_pout_lo,
    int B, int N, int resid, float eps, const float* __restrict__ offb_g, const op_t* __restrict__ gout_lo,
    const float* __restrict__ stats) {
  constexpr int LW = CC + 4, KS = CC / 16;
  constexpr int XCH = HILO ? CC / 2 : CC;   // channels per X stage fill
  extern __shared__ __attribute__((aligned(16))) op_t olds[];
  float* cbias = reinterpret_cast<float*>(olds);   // [0, CC): p, [CC, 2 CC): g
  float* gam_o = cbias + 2 * CC;
  float* gam_i = gam_o + CC;
  op_t* sWp = olds + 4 * CC * 2;
  op_t* sWg = sWp + CC * LW;
  op_t* sWpl = sWg + CC * LW;   // HILO only
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, m = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  XT* xs = reinterpret_cast<XT*>(sWg + (HILO ? 2 : 1) * CC * LW) + wid * XCH * XSP;   // this wave's X stage
  // weights -> LDS (rows are 8-byte aligned: two 8-byte stores per 16-byte load), gamma, and
  // the offsets W beta (one row per thread)
  float* mu = reinterpret_cast<float*>(xs - wid * XCH * XSP);   // the X stages, free until the tile loop
  constexpr int NT = 64 * TMO_WAVES;
  static_assert(2 * CC <= NT, "one offset row per thread");
  const int orow = tid;                   // this thread's offset row: p (< CC) or g
  const bool grow = orow >= CC, gfix = grow && offb_g != nullptr;
  opx8 rv[CC / 8];                        // g rows with offb_g: the residual of g_out (mean correction)
  float offb_v = 0.f;
  // set-up in two batches of global loads (each issued whole before its first use): the weights
  // and partials, then, while the statistics reduce, the residual rows of the mean correction
  {
    const bool meanfix = offb_g && stats;
    opx8 vp[stage_per<NT, CC, CC>()], vg[stage_per<NT, CC, CC>()];
    stage_load<NT, CC, CC>(w_pout, vp);
    stage_load<NT, CC, CC>(w_gout, vg);
    const float go = tid < CC ? lno_w[tid] : 0.f, gi = tid < CC ? lni_w[tid] : 0.f;
    float pv[stats_per<NT>()];
    if (meanfix) stats_load<NT>(stats, pv);
    if (orow < 2 * CC && gfix) offb_v = offb_g[orow - CC];
    if constexpr (HILO) {
      opx8 vl[stage_per<NT, CC, CC>()];
      stage_load<NT, CC, CC>(w_pout_lo, vl);
      stage_store<NT, CC, CC>(sWpl, LW, vl);
    }
    stage_store<NT, CC, CC>(sWp, LW, vp);
    stage_store<NT, CC, CC>(sWg, LW, vg);
    if (tid < CC) {
      gam_o[tid] = go;
      gam_i[tid] = gi;
    }
    if constexpr (CC == C)
      if (orow < 2 * CC && gfix && stats) {
#pragma unroll
        for (int c = 0; c < CC / 8; ++c) rv[c] = ld_x8(gout_lo + (orow - CC) * CC + 8 * c);
      }
    if (meanfix) stats_reduce<NT>(pv, mu, mu + PS_C);
  }
  __syncthreads();
  if (orow < 2 * CC) {
    if (gfix) {   // gate offsets from the exact g_out beta (+ the mean correction)
      if constexpr (CC == C) cbias[orow] = -LOG2E * corrected_offset_regs<true>(offb_v, rv, stats != nullptr, gam_i, mu);
    } else {      // W beta from the staged 16-bit weights (p_out with its residual under HILO)
      const op_t* w = grow ? sWg + (orow - CC) * LW : sWp + orow * LW;
      const float* bet = grow ? lni_b : lno_b;
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < CC; c += 8) {
        const opx4 wa = ld_x4(w + c), wb = ld_x4(w + c + 4);
        const opx8 w8 = {wa[0], wa[1], wa[2], wa[3], wb[0], wb[1], wb[2], wb[3]};
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += (float)w8[e] * bet[c + e];
        if constexpr (HILO) {
          if (!grow) {
            const opx4 la = ld_x4(sWpl + orow * LW + c), lb = ld_x4(sWpl + orow * LW + c + 4);
            const opx8 l8 = {la[0], la[1], la[2], la[3], lb[0], lb[1], lb[2], lb[3]};
#pragma unroll
            for (int e = 0; e < 8; ++e) acc += (float)l8[e] * bet[c + e];
          }
        }
      }
      cbias[orow] = grow ? -LOG2E * acc : acc;
    }
  }
  __syncthreads();
  if (nparts > 0) x_scale = 1.f / x_store_scale(planes_amax(amax_parts, nparts), N);   // a power of two
  const long NN = (long)N * N;
  const uint32_t ntiles = (uint32_t)B * N * N / 32;
  for (uint32_t t = blockIdx.x * TMO_WAVES + wid; t < ntiles; t += gridDim.x * TMO_WAVES) {
    asm volatile("" ::: "memory");   // the offsets are re-read from LDS each tile, not pinned in VGPRs
    const long p0 = 32l * t;                       // first pair (global index b*NN + i*N + j)
    const int b = pos_tile(t, N).b;
    const long pair = p0 + m;
    opx8 xo[KS], xi[KS];
    {
      // X[b][ch][q0 .. q0+31]: 16-byte chunk c -> channel c >> 2, pairs 8*(c & 3) ..; with HILO
      // in two fills of CC/2 channels (chunks q < CC/16 of the output-aligned order are
      // channels < CC/2).  A wave's LDS accesses complete in order, so the second fill does not
      // overtake the first one's reads.
      const XT* src = X + (long)b * CC * NN + (p0 - (long)b * NN);
      float xv[CC / 2];
#pragma unroll
      for (int half = 0; half < CC / XCH; ++half) {
#pragma unroll
        for (int k = 0; k < XCH / 16; ++k) {
          const int c = lane + 64 * k, ch = c >> 2, col = (c & 3) * 8;
          *reinterpret_cast<opx8*>(xs + ch * XSP + col) =
              *reinterpret_cast<const opx8*>(src + (long)(ch + half * XCH) * NN + col);
        }
#pragma unroll
        for (int q = half * XCH / 8; q < (half + 1) * XCH / 8; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            xv[4 * q + e] = (float)xs[(oa_channel(q, h) - half * XCH + e) * XSP + m] * x_scale;
      }
      ln_oa_gamma_to_frag<CC>(xv, h, gam_o, eps, xo);
    }
    float zr[CC / 2];
    load_row_oa<CC>(z_in + pair * CC, h, zr);
    ln_oa_gamma_to_frag<CC>(zr, h, gam_i, eps, xi);
#pragma unroll   // fully unrolled: zr[] must be indexed with constants to stay in VGPRs
    for (int ob = 0; ob < CC / 32; ++ob) {
      const op_t* wp = &sWp[(32 * ob + m) * LW];
      const op_t* wg = &sWg[(32 * ob + m) * LW];
      f32x16 P = zero16(), G = zero16();
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        P = mfma32(wfrag_oa(wp, s, h), xo[s], P);   // rows = output channel, cols = pair
        G = mfma32(wfrag_oa(wg, s, h), xi[s], G);
      }
      if constexpr (HILO) {
        const op_t* wpl = &sWpl[(32 * ob + m) * LW];
#pragma unroll
        for (int s = 0; s < KS; ++s) P = mfma32(wfrag_oa(wpl, s, h), xo[s], P);
      }
      float* orow = out + pair * CC;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int q = 4 * ob + g;
        float* dst = orow + oa_channel(q, h);
        asm volatile("" ::: "memory");   // read each group's offsets where they are used
        const f32x4 cp = *reinterpret_cast<const f32x4*>(cbias + oa_channel(q, h));
        const f32x4 cg = *reinterpret_cast<const f32x4*>(cbias + CC + oa_channel(q, h));
        f32x4 v;
        if (resid == 1) v = f32x4{zr[4 * q], zr[4 * q + 1], zr[4 * q + 2], zr[4 * q + 3]};
        if (resid == 2) v = *reinterpret_cast<const f32x4*>(dst);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float u = (P[4 * g + e] + cp[e]) * rcp_fast(1.f + exp2_fast(fmaf(G[4 * g + e], -LOG2E, cg[e])));
          v[e] = resid == 0 ? u : v[e] + u;
        }
        *reinterpret_cast<f32x4*>(dst) = v;
      }
    }
  }
}

// Contraction dispatch: 256x256 tiles from N = 448 up (enough tiles to fill the chip
// and a long enough K loop), 128x128 tiles below (at N = 384 the 256x256 tiles would be 44 %
// padding: 37.3 us against 32.4 us with 128x128 tiles).
// Rectangular form (256x256 tiles, any M, Nc multiple of 32, K multiple of 64):
// X[p][i][j] = sum_k A[p][i][k] * B[p][j][k], A [P][M][K], B [P][Nc][K], X [P][M][Nc].
// amax_parts / nparts: when nparts > 0 the output scale is x_store_scale of those operand
// maxima (the trimul's planes); otherwise `scale`.
template <typename OutT>
int launch_contract_rect(const op_t* A, const op_t* B, OutT* X, int planes, int M, int Nc, int K, float scale,
                         hipStream_t st, const float* amax_parts = nullptr, int nparts = 0) {
  if (const int rc = pf_reserve_lds((const void*)tm_contract_dma_kernel<OutT>, TMD8_LDS_BYTES,
                                    "tm_contract_dma_kernel"))
    return rc;
  const int tn = (Nc + BM2 - 1) / BM2;
  const long total = (long)planes * ((M + BM2 - 1) / BM2) * tn;
  if (total > 0x3fffffff) return pf_fail(PF_E_INVALID, "contraction: too many tiles (%ld)", total);
  // a last round of whole tiles on at most half of the CUs runs as half tiles
  const int cus = device_cus();
  const long rest = cus > 0 ? total % cus : 0;
  const long full = 2 * rest <= cus && total > cus ? total - rest : total;
  tm_contract_dma_kernel<OutT><<<(unsigned)(full + 2 * (total - full)), 64 * TMD_WAVES, TMD8_LDS_BYTES, st>>>(
      A, B, X, M, Nc, K, tn, (int)total, (int)full, scale, amax_parts, nparts);
  PF_CHECK_LAUNCH("tm_contract_dma_kernel");
  return PF_OK;
}

template <typename OutT>
int launch_contract(const op_t* opA, const op_t* opB, OutT* X, int planes, int N, float scale, hipStream_t st,
                    const float* amax_parts = nullptr, int nparts = 0) {
  if (N >= 448) return launch_contract_rect<OutT>(opA, opB, X, planes, N, N, N, scale, st, amax_parts, nparts);
  const int tpd = (N + BM - 1) / BM;
  const int total = planes * tpd * tpd;
  tm_contract_kernel<OutT><<<total, 256, 0, st>>>(opA, opB, X, N, tpd, total, scale, amax_parts, nparts);
  PF_CHECK_LAUNCH("tm_contract_kernel");
  return PF_OK;
}

// Workspace: opA, opB, X planes (op_t), then TM_MAX_PARTS floats of per-workgroup maxima, then
// the PS_WG x 128 partial sums of the mean correction.
constexpr int TM_MAX_PARTS = 1024;

template <int CC>
int trimul_run(const pf_trimul_args* a) {
  hipStream_t st = (hipStream_t)a->stream;
  const int B = a->B, N = a->N;
  const size_t planes = (size_t)B * CC * N * N;
  op_t* opA = (op_t*)a->workspace;
  op_t* opB = opA + planes;
  op_t* X = opB + planes;
  float* amax_parts = reinterpret_cast<float*>(X + planes);
  float* stats = amax_parts + TM_MAX_PARTS;
  // mean correction: exact beta offsets, the three residuals, one batch element (c_z = 128)
  const bool meanfix = CC == C && B == 1 && a->in_offsets && a->p_in_lo && a->g_in_lo && a->g_out_lo;
  if (meanfix) {
    pair_stats_kernel<<<PS_WG, 64 * PS_WAVES, 0, st>>>(a->z_in, N, a->eps, stats);
    PF_CHECK_LAUNCH("pair_stats_kernel");
  } else {
    stats = nullptr;
  }
  const float* offb = CC == C ? a->in_offsets : nullptr;
  const long positions = (long)B * N * N;
  const int cus = device_cus();
  if (cus <= 0) return pf_fail(PF_E_LAUNCH, "pf_trimul_fwd: cannot query the device");
  const int grid_proj = (int)min((long)min(cus, TM_MAX_PARTS), (positions / 32 + TMP_WAVES - 1) / TMP_WAVES);
  const int grid_out = (int)min((long)cus, (positions / 32 + TMO_WAVES - 1) / TMO_WAVES);
  {
    auto kern = a->pair_mask ? tm_proj_kernel<CC, true> : tm_proj_kernel<CC, false>;
    if (const int rc = pf_reserve_lds((const void*)kern, tmp_lds<CC>(), "tm_proj_kernel")) return rc;
    kern<<<grid_proj, 64 * tmp_waves<CC>(), tmp_lds<CC>(), st>>>(
        a->z_in, a->pair_mask, a->norm_in_w, a->norm_in_b, (const op_t*)a->p_in_w, (const op_t*)a->g_in_w, opA, opB,
        amax_parts, B, N, a->direction, a->eps, offb, (const op_t*)a->p_in_lo, (const op_t*)a->g_in_lo, stats);
    PF_CHECK_LAUNCH("tm_proj_kernel");
  }
  pf_kernel_mark(PF_TIMED_CONTRACT, st, 0);
  const int rc = launch_contract<op_t>(opA, opB, X, B * CC, N, X_STORE_SCALE, st, amax_parts, grid_proj);
  pf_kernel_mark(PF_TIMED_CONTRACT, st, 1);
  if (rc != PF_OK) return rc;
  {
    const int resid = !a->accumulate ? 0 : (a->out == a->z_in ? 1 : 2);
    bool hilo = false;
    if constexpr (CC == 128) {   // the residual weights exist for c_z = 128
      if (a->p_out_lo) {
        hilo = true;
        if (const int rc2 = pf_reserve_lds((const void*)tm_out_kernel<op_t, CC, true>, tmo_lds<CC, true>(),
                                           "tm_out_kernel"))
          return rc2;
        tm_out_kernel<op_t, CC, true><<<grid_out, 64 * TMO_WAVES, tmo_lds<CC, true>(), st>>>(
            X, X_LOAD_SCALE, amax_parts, grid_proj, a->z_in, a->out, a->norm_in_w, a->norm_in_b, a->norm_out_w,
            a->norm_out_b, (const op_t*)a->p_out_w, (const op_t*)a->g_out_w, (const op_t*)a->p_out_lo, B, N, resid,
            a->eps, offb ? offb + 4 * CC : nullptr, (const op_t*)a->g_out_lo, stats);
      }
    }
    if (!hilo) {
      if (const int rc2 = pf_reserve_lds((const void*)tm_out_kernel<op_t, CC>, tmo_lds<CC>(), "tm_out_kernel"))
        return rc2;
      tm_out_kernel<op_t, CC><<<grid_out, 64 * TMO_WAVES, tmo_lds<CC>(), st>>>(
          X, X_LOAD_SCALE, amax_parts, grid_proj, a->z_in, a->out, a->norm_in_w, a->norm_in_b, a->norm_out_w,
          a->norm_out_b, (const op_t*)a->p_out_w, (const op_t*)a->g_out_w, nullptr, B, N, resid, a->eps,
          offb ? offb + 4 * CC : nullptr, (const op_t*)a->g_out_lo, stats);
    }
    PF_CHECK_LAUNCH("tm_out_kernel");
  }
  return PF_OK;
}

}  // namespace

// ---------------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------------
extern "C" size_t pf_trimul_workspace_size(int B, int N, int C_) {
  if (B <= 0 || N <= 0 || (C_ != 128 && C_ != 64)) return 0;
  const size_t planes = (size_t)B * C_ * N * N;
  // opA, opB, X, operand maxima, mean-correction partials
  return planes * 3 * sizeof(op_t) + (TM_MAX_PARTS + PS_PARTIAL_FLOATS) * sizeof(float);
}

extern "C" int pf_trimul_fwd(const pf_trimul_args* a) {
  if (!a) return pf_fail(PF_E_INVALID, "pf_trimul_fwd: null args");
  if (a->C != 128 && a->C != 64)
    return pf_fail(PF_E_INVALID, "pf_trimul_fwd: c_z must be 128 or 64 (got %d)", a->C);
  if (a->hidden != a->C) return pf_fail(PF_E_INVALID, "pf_trimul_fwd: hidden must equal c_z (got %d, %d)", a->hidden, a->C);
  if (a->B <= 0 || a->N <= 0 || a->N % 64)
    return pf_fail(PF_E_INVALID, "pf_trimul_fwd: need B > 0 and N a positive multiple of 64 (B=%d N=%d)", a->B, a->N);
  if ((unsigned long long)a->B * a->N * a->N >= (1ull << 32))
    return pf_fail(PF_E_INVALID, "pf_trimul_fwd: B * N * N must be below 2^32 (B=%d N=%d)", a->B, a->N);
  if (a->direction != 0 && a->direction != 1)
    return pf_fail(PF_E_INVALID, "pf_trimul_fwd: direction must be 0 (outgoing) or 1 (incoming)");
  if (!a->z_in || !a->out || !a->norm_in_w || !a->norm_in_b || !a->p_in_w || !a->g_in_w ||
      !a->norm_out_w || !a->norm_out_b || !a->p_out_w || !a->g_out_w || !a->workspace)
    return pf_fail(PF_E_INVALID, "pf_trimul_fwd: null pointer argument");
  if ((a->p_out_lo || a->in_offsets || a->p_in_lo || a->g_in_lo || a->g_out_lo) && a->C != 128)
    return pf_fail(PF_E_INVALID, "pf_trimul_fwd: weight residuals and exact offsets are supported for c_z = 128 only");
  if ((a->p_in_lo || a->g_in_lo || a->g_out_lo) && !(a->in_offsets && a->p_in_lo && a->g_in_lo && a->g_out_lo))
    return pf_fail(PF_E_INVALID, "pf_trimul_fwd: the mean correction needs in_offsets, p_in_lo, g_in_lo and g_out_lo");
  const size_t need = pf_trimul_workspace_size(a->B, a->N, a->C);
  if (a->workspace_bytes < need)
    return pf_fail(PF_E_INVALID, "pf_trimul_fwd: workspace too small (%zu < %zu bytes)", a->workspace_bytes, need);
  return a->C == 128 ? trimul_run<128>(a) : trimul_run<64>(a);
}

int pf_contract_rect(const void* A, const void* B, void* X, int x_fp32, int planes, int M, int Nc, int K,
                     float scale, hipStream_t st) {
  if (!A || !B || !X) return pf_fail(PF_E_INVALID, "pf_batched_nt_gemm: null pointer");
  if (planes <= 0 || M <= 0 || Nc <= 0 || K <= 0 || M % 32 || Nc % 32 || K % 64)
    return pf_fail(PF_E_INVALID, "pf_batched_nt_gemm: need M, Nc multiples of 32 and K a multiple of 64 "
                                 "(planes=%d M=%d Nc=%d K=%d)", planes, M, Nc, K);
  if ((long)M * K >= (1l << 31) || (long)Nc * K >= (1l << 31))
    return pf_fail(PF_E_INVALID, "pf_batched_nt_gemm: a plane of A or B exceeds 2^31 elements");
  if (x_fp32) return launch_contract_rect<float>((const op_t*)A, (const op_t*)B, (float*)X, planes, M, Nc, K, scale, st);
  return launch_contract_rect<op_t>((const op_t*)A, (const op_t*)B, (op_t*)X, planes, M, Nc, K, scale, st);
}

extern "C" int pf_batched_nt_gemm(const void* A, const void* B, void* X, int x_fp32, int planes, int M, int Nc,
                                  int K, float scale, void* stream) {
  return pf_contract_rect(A, B, X, x_fp32, planes, M, Nc, K, scale, (hipStream_t)stream);
}

// Standalone contraction (the MFMA hot loop alone), for measurement and tests.
extern "C" int pf_trimul_contract(const void* opA, const void* opB, void* X, int x_fp32, int planes, int N,
                                  void* stream) {
  if (!opA || !opB || !X) return pf_fail(PF_E_INVALID, "pf_trimul_contract: null pointer");
  if (planes <= 0 || N <= 0 || N % 64)
    return pf_fail(PF_E_INVALID, "pf_trimul_contract: need planes > 0 and N a multiple of 64");
  if (x_fp32)
    return launch_contract<float>((const op_t*)opA, (const op_t*)opB, (float*)X, planes, N, 1.f,
                                  (hipStream_t)stream);
  return launch_contract<op_t>((const op_t*)opA, (const op_t*)opB, (op_t*)X, planes, N, X_STORE_SCALE,
                               (hipStream_t)stream);
}
