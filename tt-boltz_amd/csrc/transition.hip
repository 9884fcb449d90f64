// Transition (SwiGLU MLP) and row primitives for gfx950.
//
//   tr_pair_kernel   Pair transition, C = 128: LN -> fc1|fc2 (MFMA, transposed
//                    orientation) -> silu(a)*b in registers -> fc3 (MFMA) -> residual.
//                    The 4C hidden activations never leave the CU.  fc1/fc2 rows are
//                    staged in LDS perm16-permuted so the fc1/fc2 accumulator registers
//                    come out in the natural k order of fc3's B operand.  Everything is in
//                    the output-aligned layout (pf_common.h): fc3 yields D[channel][pair],
//                    so a lane owns one pair and writes 16-byte runs, and the residual is
//                    fetched with 16-byte loads, all issued before the first store.  Weight
//                    blocks arrive by LDS DMA (layout at the kernel).  fc3's rounding
//                    residual enters as a second MFMA or through a sampled mean
//                    correction (TrMode below).
//                    Replaces Transition.forward (tt_bio/boltz2.py:1227-1258) and the ttnn
//                    Transition (tt_bio/tenstorrent.py:856-946).
//   ln_rows_kernel   LayerNorm over rows, any C (nn.LayerNorm / tt_bio/boltz2.py:738-768).
//   linear_rows_kernel  out = resid + x W^T + bias, optional SwiGLU pairing of two weight
//                    matrices (tt_bio/boltz2.py:638-731); fp32 in/out, MFMA inside.
//   pair_ln_linear_kernel  out = base + W LN(x) for C = 128 rows (trunk recycling step).
#include "pf_common.h"
#include "pf_internal.h"

namespace {

constexpr int C = 128, LDSW = 136, LDS3 = 40;
PF_DEV opx8 lds_x8(const char* p) { return *reinterpret_cast<const opx8*>(p); }

// Pair transition: a workgroup is TRW waves x 32 pairs; three workgroups share a CU.
// Weight blocks of 32 hidden units move global -> LDS by DMA (global_load_lds) into a
// 2-stage ring, one barrier per block:
//   W1 / W2 block: LDS row R (0..31) holds hidden unit 32 hb + perm16(R) (so the fc1/fc2
//                  accumulator rows come out in fc3's k order); 16 chunks of 8 channels,
//                  chunk c at slot c ^ (R & 15)
//   W3 block:      row R (output channel 0..127) holds hidden 32 hb .. 32 hb + 31; 4
//                  chunks, chunk c at slot c ^ swz4(R)
// so every fragment read (one 16-byte chunk from each of 32 consecutive rows) is free of
// bank conflicts.
// The output projection fc3 comes in four forms (TrMode):
//   TR_PLAIN    fc3_16 only.
//   TR_HILO     fc3 also comes with its rounding residual w3_lo = fc3 - fc3_16 (op_t), staged
//               as a fourth block beside W3 and multiplied in as a second MFMA per fragment, so
//               the projection runs on weights good to ~2^-22 of their size; the larger ring
//               leaves room for two workgroups per CU instead of three.
//   TR_MEANFIX  fc3_16, plus corr = w3_lo . mean(h) on every output row: the part of the
//               residual's error that every position shares, h the hidden activation
//               silu(fc1 x) * fc2 x averaged over sampled positions (below).
//   TR_STATS    the sampling pass behind corr: a workgroup of 4 waves takes 4 sampled tiles of
//               32 pairs (Fibonacci hashing, as pair_stats_kernel) and two of the hidden blocks
//               (both fetched at once, before the LayerNorm: the pass is latency-bound),
//               multiplies their h by w3_lo (given as w3) and sums over its pairs into one
//               partial per workgroup (already divided by the sample size).
enum TrMode { TR_PLAIN = 0, TR_HILO = 1, TR_MEANFIX = 2, TR_STATS = 3 };
constexpr int TRW = 4;                       // waves of a workgroup
constexpr int TR_BLK = 8192;                 // bytes of one fp16 weight block
#ifndef PF_TRS_TILES
#define PF_TRS_TILES 256
#endif
constexpr int TRS_TILES = PF_TRS_TILES;      // sampled tiles of the TR_STATS pass
constexpr int TRS_MAX_HIDDEN = 512;          // its hidden sizes: multiples of 64 up to this
constexpr int TRS_PARTIALS = TRS_TILES / TRW * (TRS_MAX_HIDDEN / 64);   // its workgroups (at most)
template <int MODE>
constexpr int tr_stage() { return (MODE == TR_HILO ? 4 : 3) * TR_BLK; }
PF_DEV int tr_swz4(int r) { return (r >> 2) & 3; }

template <bool ZBIAS, int MODE>
__global__ __launch_bounds__(64 * TRW, MODE == TR_HILO || MODE == TR_STATS ? 2 : 3) void tr_pair_kernel(
    const float* x_in, float* out, const float* __restrict__ lnw, const float* __restrict__ lnb,
    const op_t* __restrict__ w1, const op_t* __restrict__ w2, const op_t* __restrict__ w3,
    const op_t* __restrict__ w3_lo, long rows, int hidden, int accumulate, float eps, ZBiasArgs zb,
    const float* __restrict__ corr, float* __restrict__ partials) {
  constexpr bool HILO = MODE == TR_HILO, STATS = MODE == TR_STATS;
  constexpr int STAGE = tr_stage<MODE>();
  __shared__ __attribute__((aligned(16))) char tl[2 * STAGE];
  __shared__ float red[STATS ? 2 * TRW * C : 1];   // the sampling pass's sums
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, m = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nhb = hidden / 32;
  long pos0;
  int hb_lo = 0, hb_hi = nhb;
  bool live = true;
  uint32_t ns = 0;
  if constexpr (STATS) {   // hidden blocks 2 hbg, 2 hbg + 1 of sampled tiles 4 g .. 4 g + 3
    const uint32_t ntiles = (uint32_t)(rows / 32);
    ns = ntiles < (uint32_t)TRS_TILES ? ntiles : (uint32_t)TRS_TILES;
    const int ngroups = nhb / 2, hbg = blockIdx.x % ngroups;
    const uint32_t k = blockIdx.x / ngroups * TRW + wid;
    live = k < ns;   // a dead wave still takes its part in the weight DMA and the barriers
    const uint32_t kk = live ? k : 0;
    pos0 = 32l * (ns == ntiles ? kk : (uint32_t)(((uint64_t)kk * 2654435761ull) % ntiles));
    hb_lo = 2 * hbg;
    hb_hi = hb_lo + 2;
  } else {
    pos0 = ((long)blockIdx.x * TRW + wid) * 32;
  }


  // DMA: chunk e = tid + 256 i (i = 0, 1) of each block; chunk tid + 256 is row R + 16
  // (W1 / W2: same slot, perm16(R + 16) = perm16(R) + 16) or R + 64 (W3: same slot)
  const int R = tid >> 4, R3 = tid >> 2;
  const uint32_t o12 = 2u * (perm16(R) * C + 8 * ((tid & 15) ^ (R & 15)));
  const uint32_t o3 = 2u * (R3 * hidden + 8 * ((tid & 3) ^ tr_swz4(R3)));
  const uint32_t o3b = 2u * 64 * hidden;
  auto issue = [&](int hb, int buf) {
    char* st = tl + buf * STAGE + 1024 * wid;
    const char* b1 = (const char*)(w1 + (long)32 * hb * C);
    const char* b2 = (const char*)(w2 + (long)32 * hb * C);
    const char* b3 = (const char*)(w3 + 32 * hb);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      __builtin_amdgcn_global_load_lds(b1 + o12 + 4096 * i, st + 4096 * i, 16, 0, 0);
      __builtin_amdgcn_global_load_lds(b2 + o12 + 4096 * i, st + TR_BLK + 4096 * i, 16, 0, 0);
      __builtin_amdgcn_global_load_lds(b3 + o3 + o3b * i, st + 2 * TR_BLK + 4096 * i, 16, 0, 0);
      if constexpr (HILO)
        __builtin_amdgcn_global_load_lds((const char*)(w3_lo + 32 * hb) + o3 + o3b * i, st + 3 * TR_BLK + 4096 * i,
                                         16, 0, 0);
    }
  };
  // fragment read addresses: fc1 / fc2 k-step s of row m; fc3 k-step ks of row 32 ob + m
  int a12[8], a3[2];
#pragma unroll
  for (int s2 = 0; s2 < 8; ++s2) a12[s2] = 256 * m + 16 * ((2 * s2 + h) ^ (m & 15));
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) a3[ks] = 2 * TR_BLK + 64 * m + 16 * ((2 * ks + h) ^ tr_swz4(m));

  // the first block (TR_STATS: both) is on its way during the LayerNorm
  issue(hb_lo, 0);
  if constexpr (STATS) issue(hb_lo + 1, 1);
  // rows past the end are clamped on load and skipped on store
  opx8 xf[8];
  {
    float x[64];
    load_row128_frag(x_in + min(pos0 + m, rows - 1) * C, h, x);
    ln128_to_frag(x, h, lnw, lnb, eps, xf);
  }
  f32x16 acc[4];
#pragma unroll
  for (int ob = 0; ob < 4; ++ob) acc[ob] = zero16();
  float cm[4];   // TR_MEANFIX: corr of channels 32 ob + m
  if constexpr (MODE == TR_MEANFIX)
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) cm[ob] = corr[32 * ob + m];

  for (int hb = hb_lo; hb < hb_hi; ++hb) {
    const int buf = (hb - hb_lo) & 1;
    __builtin_amdgcn_s_waitcnt(vmcnt_le(0));   // block hb landed ...
    __builtin_amdgcn_s_barrier();              // ... for every wave; the other stage is free
    asm volatile("" ::: "memory");
    if (!STATS && hb + 1 < hb_hi) issue(hb + 1, buf ^ 1);
    const char* st = tl + buf * STAGE;
    f32x16 a1 = zero16(), a2 = zero16();
#pragma unroll
    for (int s2 = 0; s2 < 8; ++s2) {
      a1 = mfma32(lds_x8(st + a12[s2]), xf[s2], a1);            // rows = hidden (perm16), cols = pairs
      a2 = mfma32(lds_x8(st + TR_BLK + a12[s2]), xf[s2], a2);
    }
    opx8 hf[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int t = 0; t < 8; ++t) hf[ks][t] = (op_t)(siluf(a1[8 * ks + t]) * a2[8 * ks + t]);
#pragma unroll
    for (int ob = 0; ob < 4; ++ob)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        acc[ob] = mfma32(lds_x8(st + a3[ks] + 2048 * ob), hf[ks], acc[ob]);
        if constexpr (HILO) acc[ob] = mfma32(lds_x8(st + TR_BLK + a3[ks] + 2048 * ob), hf[ks], acc[ob]);
      }
  }
  if constexpr (STATS) {
    // sums over each row of 16 lanes (16 pairs) for all 64 values first (independent DPP chains),
    // then one store per row: red[2 wid + row16 parity][channel], the 8 rows summed below
#pragma unroll
    for (int ob = 0; ob < 4; ++ob)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[ob][i] = row16_sum(acc[ob][i]);
    if ((lane & 15) == 0) {
      float* r = red + (2 * wid + ((lane >> 4) & 1)) * C + 4 * h;
#pragma unroll
      for (int ob = 0; ob < 4; ++ob)
#pragma unroll
        for (int i = 0; i < 16; ++i) r[32 * ob + 8 * (i >> 2) + (i & 3)] = live ? acc[ob][i] : 0.f;
    }
    __syncthreads();
    if (tid < C) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < 2 * TRW; ++w) sum += red[w * C + tid];
      partials[blockIdx.x * C + tid] = sum / (32.f * (float)ns);
    }
  } else {
    if constexpr (MODE == TR_MEANFIX) {
      // acc[ob] += corr on every pair, as one more MFMA: A = corr as a 16-bit hi + lo pair in
      // columns k = 0, 1 (row m = channel 32 ob + m, as for W3), B = 1; below the 16-bit
      // normal range the pair keeps corr to ~1e-8 absolute, far under the outputs' scale.
      // Accumulators that started from corr instead would keep a second copy of all 64 across
      // the loop.
      opx8 ones;
#pragma unroll
      for (int t = 0; t < 8; ++t) ones[t] = (op_t)1.f;
#pragma unroll
      for (int ob = 0; ob < 4; ++ob) {
        opx8 a;
#pragma unroll
        for (int t = 0; t < 8; ++t) a[t] = (op_t)0.f;
        const op_t hi = (op_t)(h == 0 ? cm[ob] : 0.f);
        a[0] = hi;
        a[1] = (op_t)(h == 0 ? cm[ob] - (float)hi : 0.f);
        acc[ob] = mfma32(a, ones, acc[ob]);
      }
    }
    pair_update_epilogue<ZBIAS>(acc, out, rows, pos0, m, h, accumulate, zb);
  }
}

// corr[c] = the sum of np partial rows [np][128]: one workgroup of 1024 threads, thread
// (quad q of 4 channels, group g of 32) summing rows g, g + 32, ... with all its loads in
// flight (np <= TRS_PARTIALS), then the 32 groups through LDS.
__global__ __launch_bounds__(1024) void tr_corr_kernel(const float* __restrict__ partials, int np,
                                                       float* __restrict__ corr) {
  constexpr int G = 32, PER = TRS_PARTIALS / G;
  __shared__ f32x4 part[G][C / 4 + 1];
  const int q = threadIdx.x & (C / 4 - 1), g = threadIdx.x >> 5;
  f32x4 v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int p = g + G * i;
    v[i] = p < np ? *reinterpret_cast<const f32x4*>(partials + (size_t)p * C + 4 * q) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  f32x4 sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < PER; ++i) sum += v[i];
  part[g][q] = sum;
  __syncthreads();
  if (threadIdx.x < C) {
    const int c = threadIdx.x;
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < G; ++j) t += part[j][c >> 2][c & 3];
    corr[c] = t;
  }
}

// Workspace of the C = 128 pair transition: the TR_STATS partials and corr (fp32).
constexpr size_t TR_WS_BYTES = ((size_t)TRS_PARTIALS + 1) * C * sizeof(float);

// Checks of the fc3 residual options: C = 128 only; the mean correction needs the residual and
// the workspace for its sums.
int tr_check_fc3(const pf_transition_args* a, const char* fn) {
  if (a->fc3_lo && a->C != C)
    return pf_fail(PF_E_INVALID, "%s: the fc3 residual (fc3_lo) is supported for C = 128 only", fn);
  if (a->fc3_mean_fix && !a->fc3_lo)
    return pf_fail(PF_E_INVALID, "%s: fc3_mean_fix needs the fc3 residual (fc3_lo)", fn);
  if (a->fc3_mean_fix && (a->hidden % 64 || a->hidden > TRS_MAX_HIDDEN))
    return pf_fail(PF_E_INVALID, "%s: fc3_mean_fix needs hidden a multiple of 64 up to %d (got %d)", fn,
                   TRS_MAX_HIDDEN, a->hidden);
  if (a->fc3_mean_fix && (!a->workspace || a->workspace_bytes < TR_WS_BYTES))
    return pf_fail(PF_E_INVALID, "%s: fc3_mean_fix needs a workspace of %zu bytes (got %zu)", fn, TR_WS_BYTES,
                   a->workspace ? a->workspace_bytes : (size_t)0);
  return PF_OK;
}

// The pair transition's launch over workgroups of TRW tiles of 32 pairs (the last one clamped):
// plain, hi + lo, or the mean-corrected form after its sampling pass.
template <bool ZBIAS>
int launch_tr_pair(const pf_transition_args* a, const ZBiasArgs& zb) {
  hipStream_t st = (hipStream_t)a->stream;
  const unsigned grid = (unsigned)((a->rows + 32 * TRW - 1) / (32 * TRW));
  const op_t *w1 = (const op_t*)a->fc1_w, *w2 = (const op_t*)a->fc2_w, *w3 = (const op_t*)a->fc3_w;
  const op_t* lo = (const op_t*)a->fc3_lo;
  if (lo && a->fc3_mean_fix) {
    float* partials = (float*)a->workspace;
    float* corr = partials + (size_t)TRS_PARTIALS * C;
    const long ntiles = a->rows / 32, ns = ntiles < TRS_TILES ? ntiles : TRS_TILES;
    const int np = (int)((ns + TRW - 1) / TRW) * (a->hidden / 64);
    if (ns > 0) {
      tr_pair_kernel<false, TR_STATS><<<np, 64 * TRW, 0, st>>>(a->x_in, nullptr, a->norm_w, a->norm_b, w1, w2, lo,
                                                              nullptr, a->rows, a->hidden, 0, a->eps, ZBiasArgs{},
                                                              nullptr, partials);
      PF_CHECK_LAUNCH("tr_pair_kernel (sampling pass)");
    }
    tr_corr_kernel<<<1, 1024, 0, st>>>(partials, ns > 0 ? np : 0, corr);   // no sample: corr = 0
    PF_CHECK_LAUNCH("tr_corr_kernel");
    tr_pair_kernel<ZBIAS, TR_MEANFIX><<<grid, 64 * TRW, 0, st>>>(a->x_in, a->out, a->norm_w, a->norm_b, w1, w2, w3,
                                                                nullptr, a->rows, a->hidden, a->accumulate, a->eps,
                                                                zb, corr, nullptr);
  } else if (lo) {
    tr_pair_kernel<ZBIAS, TR_HILO><<<grid, 64 * TRW, 0, st>>>(a->x_in, a->out, a->norm_w, a->norm_b, w1, w2, w3, lo,
                                                             a->rows, a->hidden, a->accumulate, a->eps, zb, nullptr,
                                                             nullptr);
  } else {
    tr_pair_kernel<ZBIAS, TR_PLAIN><<<grid, 64 * TRW, 0, st>>>(a->x_in, a->out, a->norm_w, a->norm_b, w1, w2, w3,
                                                              nullptr, a->rows, a->hidden, a->accumulate, a->eps, zb,
                                                              nullptr, nullptr);
  }
  PF_CHECK_LAUNCH("tr_pair_kernel");
  return PF_OK;
}

// Transition with C = 64, hidden = 256 (the MSA transition, tt_bio/reference.py:1333,
// boltz2.py:1188-1258), fused like the pair transition.  Persistent: one workgroup of
// 8 waves per CU keeps fc1, fc2 ([256][64]) and fc3 ([64][256]) in LDS (96 KB); a wave
// walks tiles of 32 rows: LN -> fc1|fc2 as D[hidden][row] (rows of fc1/fc2 in perm16
// order within each 32-block, so the accumulators come out in fc3's k order) ->
// silu(a)*b -> fc3 as D[channel][row] -> residual in the output-aligned layout.
// LDS rows are unpadded with XOR-swizzled 16-byte chunks (conflict-free fragment reads).
constexpr int T64_WAVES = 8;

__global__ __launch_bounds__(64 * T64_WAVES, 1) void tr64_kernel(
    const float* x_in, float* out, const float* __restrict__ lnw, const float* __restrict__ lnb,
    const op_t* __restrict__ w1, const op_t* __restrict__ w2, const op_t* __restrict__ w3, long rows,
    int accumulate, float eps) {
  __shared__ __attribute__((aligned(16))) op_t s1[256 * 64];
  __shared__ __attribute__((aligned(16))) op_t s2[256 * 64];
  __shared__ __attribute__((aligned(16))) op_t s3[64 * 256];
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, m = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  for (int c = tid; c < 256 * 8; c += 64 * T64_WAVES) {   // fc1 / fc2: 256 rows of 8 chunks
    const int R = c >> 3, k = c & 7;
    const int src = (32 * (R >> 5) + perm16(R & 31)) * 64 + 8 * k;
    const int dst = R * 64 + 8 * (k ^ swz8r(R));
    st_x8(s1 + dst, ld_x8(w1 + src));
    st_x8(s2 + dst, ld_x8(w2 + src));
  }
  for (int c = tid; c < 64 * 32; c += 64 * T64_WAVES) {   // fc3: 64 rows of 32 chunks
    const int R = c >> 5, k = c & 31;
    st_x8(s3 + R * 256 + 8 * (k ^ (R & 15)), ld_x8(w3 + R * 256 + 8 * k));
  }
  __syncthreads();
  const int sw = swz8r(m);
  const long ntiles = (rows + 31) / 32;
  for (long t = (long)blockIdx.x * T64_WAVES + wid; t < ntiles; t += (long)gridDim.x * T64_WAVES) {
    const long r0 = 32 * t;
    const long row = min(r0 + m, rows - 1);
    opx8 xf[4];
    ln64_to_frag(x_in + row * 64, h, lnw, lnb, eps, xf);
    f32x16 acc[2] = {zero16(), zero16()};
#pragma unroll 1
    for (int blk = 0; blk < 8; ++blk) {
      f32x16 a1 = zero16(), a2 = zero16();
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int off = (32 * blk + m) * 64 + 8 * ((2 * st + h) ^ sw);
        a1 = mfma32(ld_x8(s1 + off), xf[st], a1);   // rows = hidden (perm16), cols = row
        a2 = mfma32(ld_x8(s2 + off), xf[st], a2);
      }
#pragma unroll
      for (int sp = 0; sp < 2; ++sp) {
        opx8 hf;
#pragma unroll
        for (int u = 0; u < 8; ++u) hf[u] = (op_t)(siluf(a1[8 * sp + u]) * a2[8 * sp + u]);
        const int kc = 2 * (2 * blk + sp) + h;   // fc3 row chunk: hidden 32 blk + 16 sp + 8 h
#pragma unroll
        for (int ob = 0; ob < 2; ++ob) {
          const int R = 32 * ob + m;
          acc[ob] = mfma32(ld_x8(s3 + R * 256 + 8 * (kc ^ (R & 15))), hf, acc[ob]);   // rows = channel
        }
      }
    }
    if (r0 + m >= rows) continue;
    // lane (row m, h): acc[ob][4 g + e] is channel 32 ob + 8 g + 4 h + e; x_in may alias out
    const float* src = x_in + (r0 + m) * 64;
    float* dst = out + (r0 + m) * 64;
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
}

// One wave per row.
// One wave per row.  Rows of up to 64 * LN_REG values are read once into registers (all of a
// lane's loads in flight together); longer rows are read three times.
constexpr int LN_REG = 8;
__global__ __launch_bounds__(256) void ln_rows_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      const float* __restrict__ b, float* __restrict__ out,
                                                      long rows, int C_, float eps) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + row * C_;
  float* orow = out + row * C_;
  if (C_ <= 64 * LN_REG) {
    float xv[LN_REG];
#pragma unroll
    for (int u = 0; u < LN_REG; ++u) xv[u] = lane + 64 * u < C_ ? xr[lane + 64 * u] : 0.f;
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < LN_REG; ++u) s += xv[u];
    const float mean = wave_sum(s) / C_;
    float v = 0.f;
#pragma unroll
    for (int u = 0; u < LN_REG; ++u) {
      const float d = lane + 64 * u < C_ ? xv[u] - mean : 0.f;
      v += d * d;
    }
    const float rstd = rsqrtf(wave_sum(v) / C_ + eps);
#pragma unroll
    for (int u = 0; u < LN_REG; ++u) {
      const int c = lane + 64 * u;
      if (c < C_) orow[c] = (xv[u] - mean) * rstd * w[c] + b[c];
    }
    return;
  }
  float s = 0.f;
  for (int c = lane; c < C_; c += 64) s += xr[c];
  const float mean = wave_sum(s) / C_;
  float v = 0.f;
  for (int c = lane; c < C_; c += 64) { const float d = xr[c] - mean; v += d * d; }
  const float rstd = rsqrtf(wave_sum(v) / C_ + eps);
  for (int c = lane; c < C_; c += 64) orow[c] = (xr[c] - mean) * rstd * w[c] + b[c];
}

// A workgroup = one 32-row x 32-column output tile of one job; its 4 waves split the K
// steps (contiguous quarters), each wave issuing up to 8 steps of loads before their
// MFMAs, so a tile pays about one memory round trip per 8 steps of its quarter.  The
// partial accumulators meet in LDS and all 256 threads run the epilogue (4 outputs each,
// 32 consecutive columns per row).  blockIdx.z selects the job (several projections of
// the same shape in one launch).  SWIGLU: out[:, n] = silu(x W[n]) * (x W2[n]).
constexpr int LIN_SPLIT = 4;
struct LinJobs { pf_lin_job j[PF_LIN_MAX_JOBS]; };

template <bool SWIGLU>
__global__ __launch_bounds__(256) void linear_rows_kernel(LinJobs jobs, long rows, int K, int Nout) {
  __shared__ float red[LIN_SPLIT][SWIGLU ? 2 : 1][16][64];
  const pf_lin_job& jb = jobs.j[blockIdx.z];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, h = lane >> 5, m = lane & 31;
  const int n0 = blockIdx.y * 32;
  const long r0 = (long)blockIdx.x * 32;
  const float* xr = jb.x + min(r0 + m, rows - 1) * K;
  const op_t* wr = (const op_t*)jb.W + (long)(n0 + m) * K;
  const op_t* wr2 = SWIGLU ? (const op_t*)jb.W2 + (long)(n0 + m) * K : nullptr;
  const int nsteps = K >> 4, per = (nsteps + LIN_SPLIT - 1) / LIN_SPLIT;
  const int s0 = min(nsteps, wid * per), s1 = min(nsteps, s0 + per);
  f32x16 acc = zero16(), acc2 = zero16();
  for (int sg = s0; sg < s1; sg += 8) {
    opx8 af[8], wf[8], wf2[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int kk = 16 * (sg + u);
      if (sg + u < s1) {
        const f32x4 a0 = *reinterpret_cast<const f32x4*>(xr + kk + 8 * h);
        const f32x4 a1 = *reinterpret_cast<const f32x4*>(xr + kk + 8 * h + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          af[u][e] = (op_t)a0[e];
          af[u][4 + e] = (op_t)a1[e];
        }
        wf[u] = ld_x8(wr + kk + 8 * h);
        if (SWIGLU) wf2[u] = ld_x8(wr2 + kk + 8 * h);
      } else {
        af[u] = zero_x8();
        wf[u] = zero_x8();
        if (SWIGLU) wf2[u] = zero_x8();
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      acc = mfma32(af[u], wf[u], acc);
      if (SWIGLU) acc2 = mfma32(af[u], wf2[u], acc2);
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    red[wid][0][r][lane] = acc[r];
    if (SWIGLU) red[wid][1][r][lane] = acc2[r];
  }
  __syncthreads();
  // thread (wid, lane) finishes accumulator registers 4 wid .. 4 wid + 3 of lane
  const int n = n0 + m;
  const float bn = jb.bias ? jb.bias[n] : 0.f;
  float v[4], res[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * wid + i;
    float a = 0.f, a2 = 0.f;
#pragma unroll
    for (int w = 0; w < LIN_SPLIT; ++w) {
      a += red[w][0][r][lane];
      if (SWIGLU) a2 += red[w][1][r][lane];
    }
    v[i] = SWIGLU ? siluf(a) * a2 : a + bn;
    // resid may alias out: all loads ahead of the stores, so they overlap
    res[i] = !SWIGLU && jb.resid ? jb.resid[min(r0 + acc_row(r, h), rows - 1) * Nout + n] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const long row = r0 + acc_row(4 * wid + i, h);
    if (row < rows) jb.out[row * Nout + n] = v[i] + res[i];
  }
}

// out[p, :] = base[p, :] + W . LN(x[p, :]),  C = 128; W resident in LDS.  HILO: W = W + W_lo and
// LN(x) = hi + lo (16-bit each), products hi.W + lo.W + hi.W_lo (the lo.W_lo term is below
// fp32's resolution of the sum).
template <bool HILO>
__global__ __launch_bounds__(256) void pair_ln_linear_kernel(
    const float* x, const float* base, const float* __restrict__ lnw, const float* __restrict__ lnb,
    const op_t* __restrict__ W, const op_t* __restrict__ W_lo, float* out, long rows, float eps) {
  __shared__ __attribute__((aligned(16))) op_t sW[(HILO ? 2 : 1) * C * LDSW];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, h = lane >> 5, m = lane & 31;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int c = tid + 256 * q;
    st_x8(&sW[(c >> 4) * LDSW + (c & 15) * 8], ld_x8(W + (c >> 4) * C + (c & 15) * 8));
    if constexpr (HILO) st_x8(&sW[C * LDSW + (c >> 4) * LDSW + (c & 15) * 8], ld_x8(W_lo + (c >> 4) * C + (c & 15) * 8));
  }
  __syncthreads();
  const long pos0 = ((long)blockIdx.x * 4 + wid) * 32;
  if (pos0 >= rows) return;
  float xv[64];
  opx8 xf[8], xl[8];
  load_row128_frag(x + min(pos0 + m, rows - 1) * C, h, xv);
  if constexpr (HILO) {
    float sm = 0.f;
#pragma unroll
    for (int i = 0; i < 64; ++i) sm += xv[i];
    const float mean = xor32_sum(sm) * (1.f / C);
    float var = 0.f;
#pragma unroll
    for (int i = 0; i < 64; ++i) { const float d = xv[i] - mean; var += d * d; }
    const float rstd = rsqrtf(xor32_sum(var) * (1.f / C) + eps);
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int c = 16 * s + 8 * h + t;
        const float y = (xv[8 * s + t] - mean) * rstd * lnw[c] + lnb[c];
        xf[s][t] = (op_t)y;
        xl[s][t] = (op_t)(y - (float)xf[s][t]);
      }
  } else {
    ln128_to_frag(xv, h, lnw, lnb, eps, xf);
  }
#pragma unroll
  for (int ob = 0; ob < 4; ++ob) {
    f32x16 acc = zero16();
#pragma unroll
    for (int s = 0; s < 8; ++s) acc = mfma32(xf[s], ld_x8(&sW[(32 * ob + m) * LDSW + 16 * s + 8 * h]), acc);
    if constexpr (HILO) {
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        acc = mfma32(xl[s], ld_x8(&sW[(32 * ob + m) * LDSW + 16 * s + 8 * h]), acc);
        acc = mfma32(xf[s], ld_x8(&sW[C * LDSW + (32 * ob + m) * LDSW + 16 * s + 8 * h]), acc);
      }
    }
    // base may alias out: all loads ahead of the stores, so they overlap
    float res[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) res[r] = base[min(pos0 + acc_row(r, h), rows - 1) * C + 32 * ob + m];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const long p = pos0 + acc_row(r, h);
      if (p < rows) out[p * C + 32 * ob + m] = res[r] + acc[r];
    }
  }
}

}  // namespace

// ---------------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------------
extern "C" int pf_layernorm_fwd(const float* x, const float* w, const float* b, float* out, long rows,
                                int C_, float eps, void* stream) {
  if (!x || !w || !b || !out) return pf_fail(PF_E_INVALID, "pf_layernorm_fwd: null pointer");
  if (rows <= 0 || C_ <= 0 || C_ > 4096) return pf_fail(PF_E_INVALID, "pf_layernorm_fwd: bad shape rows=%ld C=%d", rows, C_);
  ln_rows_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, (hipStream_t)stream>>>(x, w, b, out, rows, C_, eps);
  PF_CHECK_LAUNCH("ln_rows_kernel");
  return PF_OK;
}

int pf_linear_batch(const pf_lin_job* jobs, int njobs, long rows, int K, int Nout, hipStream_t st) {
  if (njobs < 1 || njobs > PF_LIN_MAX_JOBS) return pf_fail(PF_E_INVALID, "pf_linear_fwd: %d jobs", njobs);
  if (rows <= 0 || K <= 0 || K % 16 || Nout <= 0 || Nout % 32)
    return pf_fail(PF_E_INVALID, "pf_linear_fwd: need rows > 0, K %% 16 == 0, Nout %% 32 == 0 (rows=%ld K=%d Nout=%d)",
                   rows, K, Nout);
  LinJobs J{};
  const bool swiglu = jobs[0].W2 != nullptr;
  for (int i = 0; i < njobs; ++i) {
    if (!jobs[i].x || !jobs[i].W || !jobs[i].out) return pf_fail(PF_E_INVALID, "pf_linear_fwd: null pointer");
    if ((jobs[i].W2 != nullptr) != swiglu) return pf_fail(PF_E_INVALID, "pf_linear_fwd: mixed SwiGLU jobs");
    J.j[i] = jobs[i];
  }
  dim3 grid((unsigned)((rows + 31) / 32), (unsigned)(Nout / 32), (unsigned)njobs);
  if (swiglu)
    linear_rows_kernel<true><<<grid, 256, 0, st>>>(J, rows, K, Nout);
  else
    linear_rows_kernel<false><<<grid, 256, 0, st>>>(J, rows, K, Nout);
  PF_CHECK_LAUNCH("linear_rows_kernel");
  return PF_OK;
}

static int launch_linear(const float* x, const void* W, const void* W2, const float* bias, const float* resid,
                         float* out, long rows, int K, int Nout, hipStream_t st) {
  const pf_lin_job job{x, W, W2, bias, resid, out};
  return pf_linear_batch(&job, 1, rows, K, Nout, st);
}

extern "C" int pf_linear_fwd(const float* x, const void* W, const float* bias, const float* resid, float* out,
                             long rows, int K, int Nout, void* stream) {
  return launch_linear(x, W, nullptr, bias, resid, out, rows, K, Nout, (hipStream_t)stream);
}

extern "C" size_t pf_transition_workspace_size(long rows, int C_, int hidden) {
  if (rows <= 0 || C_ <= 0 || hidden <= 0) return 0;
  if (C_ == C && hidden % 32 == 0) return TR_WS_BYTES;   // fused pair kernel: the mean-correction sums
  if (C_ == 64 && hidden == 256) return 0;      // fused C = 64 kernel: no scratch
  return (size_t)rows * (C_ + hidden) * sizeof(float);
}

extern "C" int pf_transition_fwd(const pf_transition_args* a) {
  if (!a) return pf_fail(PF_E_INVALID, "pf_transition_fwd: null args");
  if (a->rows <= 0 || a->C <= 0 || a->hidden <= 0 || a->hidden % 32 || a->C % 32)
    return pf_fail(PF_E_INVALID, "pf_transition_fwd: need rows > 0 and C, hidden multiples of 32 (C=%d hidden=%d)",
                   a->C, a->hidden);
  if (!a->x_in || !a->out || !a->norm_w || !a->norm_b || !a->fc1_w || !a->fc2_w || !a->fc3_w)
    return pf_fail(PF_E_INVALID, "pf_transition_fwd: null pointer argument");
  hipStream_t st = (hipStream_t)a->stream;
  if (const int rc = tr_check_fc3(a, "pf_transition_fwd")) return rc;
  if (a->C == C) return launch_tr_pair<false>(a, ZBiasArgs{});
  if (a->C == 64 && a->hidden == 256) {
    const int cus = device_cus();
    if (cus <= 0) return pf_fail(PF_E_LAUNCH, "tr64_kernel: cannot query the device");
    const long tiles = (a->rows + 31) / 32;
    const int grid = (int)min((long)cus, (tiles + T64_WAVES - 1) / T64_WAVES);
    tr64_kernel<<<grid, 64 * T64_WAVES, 0, st>>>(a->x_in, a->out, a->norm_w, a->norm_b, (const op_t*)a->fc1_w,
                                                 (const op_t*)a->fc2_w, (const op_t*)a->fc3_w, a->rows,
                                                 a->accumulate, a->eps);
    PF_CHECK_LAUNCH("tr64_kernel");
    return PF_OK;
  }
  const size_t need = pf_transition_workspace_size(a->rows, a->C, a->hidden);
  if (!a->workspace || a->workspace_bytes < need)
    return pf_fail(PF_E_INVALID, "pf_transition_fwd: workspace too small (%zu < %zu bytes)", a->workspace_bytes, need);
  float* xn = (float*)a->workspace;
  float* hid = xn + (size_t)a->rows * a->C;
  int rc = pf_layernorm_fwd(a->x_in, a->norm_w, a->norm_b, xn, a->rows, a->C, a->eps, a->stream);
  if (rc) return rc;
  rc = launch_linear(xn, a->fc1_w, a->fc2_w, nullptr, nullptr, hid, a->rows, a->C, a->hidden, st);
  if (rc) return rc;
  return launch_linear(hid, a->fc3_w, nullptr, nullptr, a->accumulate ? a->out : nullptr, a->out, a->rows,
                       a->hidden, a->C, st);
}

extern "C" int pf_pair_ln_linear_fwd(const float* x, const float* base, const float* ln_w, const float* ln_b,
                                     const void* W, const void* W_lo, float* out, long rows, int C_, float eps,
                                     void* stream) {
  if (!x || !base || !ln_w || !ln_b || !W || !out) return pf_fail(PF_E_INVALID, "pf_pair_ln_linear_fwd: null pointer");
  if (C_ != C || rows <= 0) return pf_fail(PF_E_INVALID, "pf_pair_ln_linear_fwd: only C = 128 (got %d)", C_);
  if (W_lo)
    pair_ln_linear_kernel<true><<<(unsigned)((rows + 127) / 128), 256, 0, (hipStream_t)stream>>>(
        x, base, ln_w, ln_b, (const op_t*)W, (const op_t*)W_lo, out, rows, eps);
  else
    pair_ln_linear_kernel<false><<<(unsigned)((rows + 127) / 128), 256, 0, (hipStream_t)stream>>>(
        x, base, ln_w, ln_b, (const op_t*)W, nullptr, out, rows, eps);
  PF_CHECK_LAUNCH("pair_ln_linear_kernel");
  return PF_OK;
}

__global__ __launch_bounds__(256) void add_kernel(const float* a, const float* b, float* out, long n) {
  const long n4 = n / 4, stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const f32x4 u = reinterpret_cast<const f32x4*>(a)[i], v = reinterpret_cast<const f32x4*>(b)[i];
    reinterpret_cast<f32x4*>(out)[i] = u + v;
  }
  for (long i = 4 * n4 + (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = a[i] + b[i];
}

extern "C" int pf_add_fwd(const float* a, const float* b, float* out, long n, void* stream) {
  if (!a || !b || !out) return pf_fail(PF_E_INVALID, "pf_add_fwd: null pointer");
  if (n <= 0) return pf_fail(PF_E_INVALID, "pf_add_fwd: n = %ld", n);
  if (((uintptr_t)a | (uintptr_t)b | (uintptr_t)out) & 15)
    return pf_fail(PF_E_INVALID, "pf_add_fwd: pointers must be 16-byte aligned");
  const int cus = device_cus();
  if (cus <= 0) return pf_fail(PF_E_LAUNCH, "pf_add_fwd: cannot query the device");
  const long blocks = min((long)cus * 8, (n / 4 + 255) / 256 + 1);
  add_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(a, b, out, n);
  PF_CHECK_LAUNCH("add_kernel");
  return PF_OK;
}

extern "C" int pf_transition_pair_bias_fwd(const pf_transition_args* a, const pf_apb_args* apb) {
  if (!a || !apb) return pf_fail(PF_E_INVALID, "pf_transition_pair_bias_fwd: null args");
  if (a->C != C || a->hidden <= 0 || a->hidden % 32)
    return pf_fail(PF_E_INVALID, "pf_transition_pair_bias_fwd: need C = 128 and hidden a multiple of 32 (C=%d hidden=%d)",
                   a->C, a->hidden);
  if (!a->x_in || !a->out || !a->norm_w || !a->norm_b || !a->fc1_w || !a->fc2_w || !a->fc3_w)
    return pf_fail(PF_E_INVALID, "pf_transition_pair_bias_fwd: null pointer argument");
  pf_apb_args chk = *apb;
  chk.z = a->out;   // the bias is computed from the transition's output
  int rc = pf_apb_check(&chk, "pf_transition_pair_bias_fwd", true);
  if (rc) return rc;
  if ((rc = tr_check_fc3(a, "pf_transition_pair_bias_fwd"))) return rc;
  if (a->fc3_mean_fix) {   // the sums must survive the bias writes of the same launch
    const char *t0 = (const char*)a->workspace, *b0 = (const char*)apb->workspace;
    if (t0 < b0 + apb->workspace_bytes && b0 < t0 + TR_WS_BYTES)
      return pf_fail(PF_E_INVALID, "pf_transition_pair_bias_fwd: the transition workspace overlaps the attention's");
  }
  const long NN = (long)apb->N * apb->N;
  if (a->rows != (long)apb->B * NN)
    return pf_fail(PF_E_INVALID, "pf_transition_pair_bias_fwd: rows %ld != B*N*N = %ld", a->rows, (long)apb->B * NN);
  const ZBiasArgs zb{apb->zln_w, apb->zln_b, (const op_t*)apb->w_z, pf_apb_bias_ptr(apb), NN, apb->H, apb->eps};
  return launch_tr_pair<true>(a, zb);   // N % 32 == 0: whole 32-pair tiles
}
