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
//              Q, K    op_t [B][N(row i)][H][N(j)][D]
//              Vt      op_t [B][N(row i)][H][D][N(k)], keys stored at perm16(k) (bits 2
//                      and 3 swapped) so a P.V operand fragment is one 16-byte run
//              bias32  fp32 [B][H][N(j)][N(k)]   (shared by all rows i)
//              mask16  op_t [B][N(i)][N(k)]      0, or -inf for masked / padding keys
//   ta_attn  flash attention (see the kernel's comment): 16-wave workgroups of 4 frame rows
//            x 128 queries, LDS-DMA ring, bias / mask / reference max folded into MFMAs,
//            lazy-max softmax.  Output O (normalized, ungated) op_t [B][N(i)][N(j)][H*D].
//   ta_out   o-proj epilogue (persistent, W_g / W_o in LDS, output-aligned layout): gate
//            recomputed from LN(z) (MFMA), o*sigmoid(g) built in registers as linear_o's B
//            operand, residual added to the z values the lane loaded for the LayerNorm.
#include <type_traits>

#include "pf_common.h"
#include "pf_internal.h"

namespace {

// C = H * D: the attention width (q / k / v / o channels).  The pair width c_z (CC in the
// projection kernels) is 128 in the trunk and 64 in the template stack.
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

// Additive mask term of one (row, key), log2 units: -inf for padding keys and for the
// reference's 1e9*(mask-1) whenever that is beyond op_t's range (a masked key).
PF_DEV op_t mask_term(bool pad, float mv) {
  const float t = 1e9f * (mv - 1.f) * LOG2E;
  return (op_t)(pad || t < -65504.f ? -INFINITY : t);
}

// ---------------------------------------------------------------------------------
// Projection (persistent): one workgroup of 8 waves per CU keeps W_q, W_k, W_v and the
// bias rows in LDS with the LayerNorm affine folded in (W' = W diag(gamma) in op_t,
// c = W beta in fp32 as the accumulator start), so a tile only normalizes.  Each wave
// walks tiles of 32 frame positions (ip, j0 .. j0+31) and loads the next tile's z rows
// while it computes the current one.  The MFMA orientation is chosen per output so that
// the stores are 16-byte runs (8-byte runs write at ~2/3 of the bandwidth):
//   Q, K  [j][d]:  D[d][pos]   runs of 4 d, paired across lane halves (store_runs16)
//   V^T   [d][k]:  D[pos][d]   a lane's key runs g = 2p, 2p+1 are 8 adjacent slots
//   bias  [hd][j]: D[hd][pos]  a lane holds the 4 heads of its position
// FAST (the fast mode's block-fp8 points): q, k and v are quantize-dequantized per head (one
// 32-channel block per position) before they are stored.  Q and K blocks are lane pairs of
// the D[d][pos] accumulator; V's D[pos][d] orientation spreads a block over 32 lanes, so a
// D[d][pos] copy of V gives each key's block scale, passed through 32 floats of LDS per wave.
// ---------------------------------------------------------------------------------
constexpr int TAP_WAVES = 8;
constexpr int TAP_ROWS = 3 * C + 32;   // q, k, v rows, then 32 bias rows (H used, rest zero)
// LDS: the weights [TAP_ROWS][CC + 8] op_t, their accumulator starts [TAP_ROWS] fp32, then (FAST)
// the per-wave V block scales or the mean-correction mu [128] and its reduction scratch (the two
// never coexist)
template <int CC, bool FAST = false>
constexpr size_t tap_lds() {
  return (size_t)TAP_ROWS * (CC + 8) * sizeof(op_t) + TAP_ROWS * sizeof(float) +
         (FAST ? TAP_WAVES * 32 * sizeof(float) : (PS_C + 64 * TAP_WAVES) * sizeof(float));
}

// offb (optional, fp32 [3 C + H]): the exact W beta of the q, k, v and bias rows (else computed
// from the op_t weights); with lo (the residuals of the kernel's gamma-folded weights, W diag(gamma)
// - op_t(W16 diag(gamma)), four [rows][CC] arrays for q, k, v, bias) and the stats partials also
// the mean correction of those weights (see pair_stats_kernel).
struct TaMeanFix { const float* offb; const op_t* lo[4]; const float* stats; };

template <int CC, bool FAST>
__global__ __launch_bounds__(64 * TAP_WAVES, 1) void ta_proj_kernel(
    const float* __restrict__ z, const float* __restrict__ pair_mask,
    const float* __restrict__ lnw, const float* __restrict__ lnb,
    const op_t* __restrict__ wq, const op_t* __restrict__ wk, const op_t* __restrict__ wv,
    const op_t* __restrict__ wb, op_t* __restrict__ Q, op_t* __restrict__ K,
    op_t* __restrict__ Vt, float* __restrict__ bias32, op_t* __restrict__ mask16,
    int B, int N, int n_valid, int ending, float qscale, float eps, TaMeanFix mf) {
  constexpr int LW = CC + 8, KS = CC / 16;
  extern __shared__ __attribute__((aligned(16))) op_t plds[];
  float* cb = reinterpret_cast<float*>(plds + TAP_ROWS * LW);
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, m = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  float* vsc = cb + TAP_ROWS + 32 * wid;   // FAST: this wave's per-key V block scales
  float* mu = cb + TAP_ROWS;               // !FAST: the mean correction's mu
  auto wrow = [&](int row) -> const op_t* {   // weight rows have CC inputs
    return row < C ? wq + row * CC : row < 2 * C ? wk + (row - C) * CC
         : row < 3 * C ? wv + (row - 2 * C) * CC : wb + (row - 3 * C) * CC;
  };
  {   // every global load of the set-up first (weights, the offset row, partials), then LDS
    constexpr int NT = 64 * TAP_WAVES, CH = TAP_ROWS * (CC / 8), SPER = (CH + NT - 1) / NT;
    static_assert(TAP_ROWS <= NT && NT % (CC / 8) == 0, "one offset row per thread; one column per thread");
    const int col = (tid % (CC / 8)) * 8;   // the same for every chunk of this thread
    opx8 wv[SPER];
#pragma unroll
    for (int i = 0; i < SPER; ++i) {
      const int c = tid + NT * i, row = c / (CC / 8);
      wv[i] = c < CH && row < 3 * C + H ? ld_x8(wrow(row) + col) : zero_x8();
    }
    float gcol[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) gcol[e] = lnw[col + e];
    const bool meanfix = !FAST && mf.offb && mf.stats;
    const int orow = tid;   // this thread's offset row
    const bool live_row = orow < 3 * C + H;
    float pv[stats_per<NT>()];
    if (meanfix) stats_load<NT>(mf.stats, pv);
    // the row behind this thread's offset: the residual (mean correction) or the weight (W beta)
    opx8 rv[CC / 8];
    float offb_v = 0.f;
    const bool use_offb = !FAST && mf.offb;
    if (live_row) {
      if (use_offb) {
        offb_v = mf.offb[orow];
        if constexpr (CC == PS_C)
          if (mf.stats) {
            const op_t* lo = mf.lo[orow < 3 * C ? orow / C : 3] + (orow < 3 * C ? orow % C : orow - 3 * C) * CC;
#pragma unroll
            for (int c = 0; c < CC / 8; ++c) rv[c] = ld_x8(lo + 8 * c);
          }
      } else {
        const op_t* w = wrow(orow);
#pragma unroll
        for (int c = 0; c < CC / 8; ++c) rv[c] = ld_x8(w + 8 * c);
      }
    }
#pragma unroll
    for (int i = 0; i < SPER; ++i) {
      const int c = tid + NT * i, row = c / (CC / 8);
      if (c < CH) {
        opx8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (op_t)((float)wv[i][e] * gcol[e]);
        st_x8(plds + row * LW + col, row < 3 * C + H ? v : zero_x8());
      }
    }
    if (meanfix) {
      stats_reduce<NT>(pv, mu, mu + PS_C);
      __syncthreads();
    }
    if (orow < TAP_ROWS) {   // accumulator starts W beta
      float acc = 0.f;
      if (live_row) {
        if (use_offb) {
          if constexpr (CC == PS_C) acc = corrected_offset_regs<false>(offb_v, rv, mf.stats != nullptr, nullptr, mu);
        } else {
#pragma unroll
          for (int c = 0; c < CC / 8; ++c)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc += (float)rv[c][e] * lnb[8 * c + e];
        }
      }
      cb[orow] = acc;
    }
  }
  __syncthreads();

  const uint32_t tiles = (uint32_t)B * N * N / 32;
  const uint32_t stride = gridDim.x * TAP_WAVES;
  // frame tile t -> (b, ip, j0) and the z pair this lane's row comes from
  auto decode = [&](uint32_t t, int& b, int& ip, int& j0) PF_INLINE {
    const PosTile pt = pos_tile(t, N);
    b = pt.b;
    ip = pt.r;
    j0 = pt.c0;
  };
  auto zpair = [&](int b, int ip, int j0) -> long {
    return ((long)b * N + (ending ? j0 + m : ip)) * N + (ending ? ip : j0 + m);
  };
  float xn[CC / 2];
  uint32_t t = blockIdx.x * TAP_WAVES + wid;
  if (t < tiles) {
    int b, ip, j0;
    decode(t, b, ip, j0);
    load_row_frag<CC>(z + zpair(b, ip, j0) * CC, h, xn);
  }
  for (; t < tiles; t += stride) {
    int b, ip, j0;
    decode(t, b, ip, j0);
    const long pair = zpair(b, ip, j0);
    opx8 xf[KS];
    {
      float x[CC / 2];
#pragma unroll
      for (int i = 0; i < CC / 2; ++i) x[i] = xn[i];
      if (t + stride < tiles) {   // next tile's rows, in flight during this tile
        int b2, ip2, j02;
        decode(t + stride, b2, ip2, j02);
        load_row_frag<CC>(z + zpair(b2, ip2, j02) * CC, h, xn);
      }
      ln_norm_to_frag<CC>(x, eps, xf);
    }
    if (h == 0) {
      // frame key j0+m of row ip: padding -> excluded; otherwise inf*(mask-1) (log2 units)
      const float mv = pair_mask ? pair_mask[pair] : 1.f;
      mask16[((long)b * N + ip) * N + j0 + m] = mask_term(j0 + m >= n_valid, mv);
    }
    const long rowh = ((long)b * N + ip) * H;   // (b, ip) head-block index base
    // Q, K: D[d][pos]; lane (pos m, h) holds d = 8g + 4h + e in acc[4g + e]
#pragma unroll 1
    for (int blk = 0; blk < 8; ++blk) {
      f32x16 acc;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 c4 = *reinterpret_cast<const f32x4*>(cb + 32 * blk + 8 * g + 4 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[4 * g + e] = c4[e];
      }
#pragma unroll
      for (int s2 = 0; s2 < KS; ++s2) acc = mfma32(ld_x8(plds + (32 * blk + m) * LW + 16 * s2 + 8 * h), xf[s2], acc);
      if constexpr (FAST) mx_fake_quant16(acc);
      op_t* dst = blk < 4 ? Q : K;
      store_runs16(dst + ((rowh + (blk & 3)) * N + j0 + m) * D, acc, blk < 4 ? qscale : 1.f, h);
    }
    // V^T: D[pos][d]; lane (d m, h) holds keys j0 + 8g + 4h + e in acc[4g + e]
#pragma unroll 1
    for (int hd = 0; hd < H; ++hd) {
      if constexpr (FAST) {   // block scale of key j0 + m -> vsc[m]
        f32x16 at;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 c4 = *reinterpret_cast<const f32x4*>(cb + 2 * C + 32 * hd + 8 * g + 4 * h);
#pragma unroll
          for (int e = 0; e < 4; ++e) at[4 * g + e] = c4[e];
        }
#pragma unroll
        for (int s2 = 0; s2 < KS; ++s2)
          at = mfma32(ld_x8(plds + (2 * C + 32 * hd + m) * LW + 16 * s2 + 8 * h), xf[s2], at);
        float a = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) a = fmaxf(a, fabsf(at[r]));
        a = xor32_max(a);
        if (h == 0) vsc[m] = mx_block_scale(a);
      }
      const float c0 = cb[2 * C + 32 * hd + m];
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = c0;
#pragma unroll
      for (int s2 = 0; s2 < KS; ++s2)
        acc = mfma32(xf[s2], ld_x8(plds + (2 * C + 32 * hd + m) * LW + 16 * s2 + 8 * h), acc);
      if constexpr (FAST) {   // same wave: its LDS accesses complete in order
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 X4 = *reinterpret_cast<const f32x4*>(vsc + 8 * g + 4 * h);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[4 * g + e] = mx_fake_quant1(acc[4 * g + e], X4[e], 448.f * X4[e]);
        }
      }
      // keys 8g + 4h + e of runs g = 2p, 2p+1 sit at storage 16p + 8h .. +7 (perm16)
      op_t* row = Vt + ((rowh + hd) * D + m) * (long)N + j0;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        opx8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (op_t)acc[8 * p + e];
        st_x8(row + 16 * p + 8 * h, v);
      }
    }
    // bias: D[hd][pos]; rows 0..H-1 are acc[0..3] of the h = 0 lanes
    {
      f32x16 acc;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 c4 = *reinterpret_cast<const f32x4*>(cb + 3 * C + 8 * g + 4 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[4 * g + e] = c4[e];
      }
#pragma unroll
      for (int s2 = 0; s2 < KS; ++s2) acc = mfma32(ld_x8(plds + (3 * C + m) * LW + 16 * s2 + 8 * h), xf[s2], acc);
      if (h == 0) {
#pragma unroll
        for (int r = 0; r < H; ++r) bias32[(((long)b * H + r) * N + ip) * N + j0 + m] = acc[r] * LOG2E;
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Flash attention.  OUT_F32 = false: O op_t [B][N][N][H*D] (frame pair layout);
// OUT_F32 = true: O fp32 [B][N][H][N][D] (the standalone attention-core API).
//
// A workgroup is 16 waves (four per SIMD): 4 frame rows (ip0 .. ip0+3) x 4 blocks of 32 queries;
// each wave owns one row and one 32-query block and walks 4 heads x N/64 key tiles.  Per step
// the workgroup's fp32 bias tile [128 q][64 k], the four rows' K [64 k][32 d] and V^T
// [32 d][64 k] tiles and their mask entries move global -> LDS by DMA (buffer loads straight to
// LDS, no VGPR staging) through a 2-deep ring, one barrier per step.  Scores S'^T[key][query]
// come out of three MFMAs per 32x32 tile:
//     bias^T (fp32, the accumulator's start value, read from LDS in accumulator order)
//     + K.Q^T (2)  +  [1, mask[key]] . [-m[q], 1]^T (1: two used k-slots)
// so the bias, the key mask and the reference max cost no VALU and the bias is not rounded;
// the softmax is exp2, an fp16 pair pack and v_dot2 row sums.  The reference max m[q] is kept
// as an op_t value (exact as an MFMA operand) and moves lazily: at a head's first tile, while a
// query has seen no unmasked key, or when a tile's row sum exceeds 2^14 (some P above 2^9).  A P
// that would overflow op_t fails the same test before it reaches the P.V MFMA, and the tile is
// then repacked from S' with the new reference.  A wave's two key halves of a step are processed
// one after the other (so a tile's scores always use the reference the previous tile left);
// four waves per SIMD (about 100 VGPRs each) hide each other's MFMA and LDS latencies.
// Rows whose valid keys are all masked: the fp32 reference adds -1e9 to every logit,
// which rounds them all to -1e9 (|logit| < 32), i.e. a uniform average over the keys.
// Such a row's waves skip the tiles (still taking part in every barrier and DMA) and write
// the mean of v after the loop.
// ---------------------------------------------------------------------------------
constexpr int TA_WAVES = 16;
// LDS sections (bytes), each holding stage 0 then stage 1:
//   bias fp32 [128 q][64 k]: rows of 256 B, 16-byte chunk c of row q at position c ^ (q & 15)
//   K   op_t  [4 rows][64 k][32 d]: rows of 64 B, chunk swizzle swz4
//   V^T op_t  [4 rows][32 d][64 k]: rows of 128 B, chunk swizzle swz8
//   mask op_t [4 rows][64 k] (wave 0's 1 KB DMA; the upper 512 B repeat the lower)
constexpr int TS_BIAS = 0, TB_STAGE = 32768;
constexpr int TS_K = 65536, TK_STAGE = 16384;
constexpr int TS_V = 98304, TV_STAGE = 16384;
constexpr int TS_MASK = 131072, TM_STAGE = 1024;
constexpr size_t TA_LDS = (size_t)TS_MASK + 2 * TM_STAGE;
constexpr float LSTEP_MAX = 16384.f;   // per-lane row sum of one tile that forces a rescale

// 16-byte chunk swizzles: rows of 8 chunks (V^T) and of 4 chunks (K).  A fragment read takes
// one chunk from each of 32 consecutive rows; any 16 consecutive rows land in 16 distinct
// 16-byte bank groups.
PF_DEV int swz8(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }
PF_DEV int swz4(int r) { return (r >> 2) & 3; }
PF_DEV opx8 lds_x8(const char* p) { return *reinterpret_cast<const opx8*>(p); }
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
PF_DEV uint32_t half_bits(op_t v) { return __builtin_bit_cast(uint16_t, v); }
PF_DEV opx8 as_x8(const u32x4& v) { return __builtin_bit_cast(opx8, v); }
// operand whose slots 0 and 1 are (lo, hi) in lanes 0..31 and zero elsewhere
PF_DEV opx8 slots01(int h, uint32_t lo_hi) {
  const u32x4 v = {h ? 0u : lo_hi, 0u, 0u, 0u};
  return as_x8(v);
}
// LDS reads from absolute LDS byte addresses (the per-lane address registers already hold the
// allocation base, so the loop's reads need no address arithmetic beyond the immediate offset)
typedef __attribute__((address_space(3))) const char* lds_ptr;
PF_DEV lds_ptr lds_at(uint32_t a) { return (lds_ptr)(uintptr_t)a; }
PF_DEV opx8 lds_rd8(uint32_t a) { return *reinterpret_cast<__attribute__((address_space(3))) const opx8*>(lds_at(a)); }
PF_DEV f32x4 lds_rd4f(uint32_t a) {
  return *reinterpret_cast<__attribute__((address_space(3))) const f32x4*>(lds_at(a));
}
PF_DEV uint32_t lds_rd16(uint32_t a) {
  return *reinterpret_cast<__attribute__((address_space(3))) const uint16_t*>(lds_at(a));
}
// Raw buffer resource over `bytes` bytes at `p` (stride 0, reads beyond `bytes` return zero).
PF_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* p, long bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)min(bytes, 0x7fffffffl), 0x00020000);
}
// 16 bytes per lane from resource byte offset voff + soff into LDS at lds + 16 * lane.
PF_DEV void dma16(__amdgpu_buffer_rsrc_t r, char* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

template <bool OUT_F32>
__global__ __launch_bounds__(64 * TA_WAVES, 1) void ta_attn_kernel(
    const op_t* __restrict__ Q, const op_t* __restrict__ K, const op_t* __restrict__ Vt,
    const float* __restrict__ bias32, const op_t* __restrict__ mask16, op_t* __restrict__ O16,
    float* __restrict__ O32, int N, int n_valid, int total, int full, int split) {
  extern __shared__ __attribute__((aligned(16))) char alds[];
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, m = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row = wid & 3, qb = wid >> 2;   // frame row, 32-query block
  // Workgroups 0 .. full-1 take all heads of their (rows, queries) block; the blocks after them
  // (a last round that would leave at least half of the CUs idle, or a whole launch that small)
  // go to `split` (2 or 4) workgroups each, H / split heads apiece, so that round takes about
  // 1 / split as long.
  int w, h0 = 0, nh = H;
  if ((int)blockIdx.x < full) {
    w = xcd_remap(blockIdx.x, full);
  } else {
    const int hw = xcd_remap(blockIdx.x - full, split * (total - full));
    w = full + hw / split;
    nh = H / split;
    h0 = (hw % split) * nh;
  }
  const int nQP = (N + 127) >> 7, nKB = N >> 6, T = nh * nKB;
  const int per_b = (N >> 2) * nQP;
  const int b = w / per_b;
  const int rem = w - b * per_b;
  const int rg = rem / nQP;
  const int jw0 = (rem - rg * nQP) * 128;
  const int ip0 = 4 * rg, ip = ip0 + row;
  const long NN = (long)N * N;
  const int seqD = N * D;                 // elements of one (row, head) Q / K / V^T block

  // ---- DMA: buffer resources (SGPRs) over this workgroup's operands, per-lane 32-bit source
  // offsets, the step's offset as the uniform soffset; reads outside a resource return 0 ----
  // bias: wave w's instruction j fills LDS bytes 2048 w + 1024 j .. of the stage, i.e. rows
  // q = 8 w + 4 j + (lane >> 4), position lane & 15, which holds chunk (lane & 15) ^ (q & 15).
  // K and V^T: chunk tid of the 16 KB tile (one instruction each); mask: wave 0, 1 KB.
  const __amdgpu_buffer_rsrc_t rB = make_rsrc(bias32 + (long)b * H * NN, (long)H * NN * 4);
  const __amdgpu_buffer_rsrc_t rK = make_rsrc(K + ((long)b * N + ip0) * H * seqD, 4l * H * seqD * 2);
  const __amdgpu_buffer_rsrc_t rV = make_rsrc(Vt + ((long)b * N + ip0) * H * seqD, 4l * H * seqD * 2);
  const __amdgpu_buffer_rsrc_t rM = make_rsrc(mask16 + ((long)b * N + ip0) * N, 4l * N * 2);
  uint32_t offB[2], offK, offV;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int q = 8 * wid + 4 * j + (lane >> 4);
    offB[j] = 4u * ((uint32_t)min(jw0 + q, N - 1) * (uint32_t)N + 4u * (uint32_t)((lane & 15) ^ (q & 15)));
  }
  {
    const int c = tid;
    const int rk = c >> 8, kk = (c >> 2) & 63, dd = (c >> 3) & 31;
    offK = 2u * (rk * H * seqD + kk * D + 8 * ((c & 3) ^ swz4(kk)));
    offV = 2u * (rk * H * seqD + dd * N + 8 * ((c & 7) ^ swz8(dd)));
  }
  const uint32_t offM = 2u * (((lane >> 3) & 3) * N + 8 * (lane & 7));
  // stage `s` of step (hd, kb0)
  auto issue = [&](int s, int hd, int kb0) PF_INLINE {
    const uint32_t sb = 4u * ((uint32_t)hd * (uint32_t)NN + (uint32_t)kb0);
    const uint32_t skv = 2u * ((uint32_t)(hd * seqD) + (uint32_t)kb0 * D);
    const uint32_t sv = 2u * ((uint32_t)(hd * seqD) + (uint32_t)kb0);
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(rB, alds + TS_BIAS + s * TB_STAGE + 2048 * wid + 1024 * j, offB[j], sb);
    dma16(rK, alds + TS_K + s * TK_STAGE + 1024 * wid, offK, skv);
    dma16(rV, alds + TS_V + s * TV_STAGE + 1024 * wid, offV, sv);
    if (wid == 0) dma16(rM, alds + TS_MASK + s * TM_STAGE, offM, 2u * (uint32_t)kb0);
  };

  // ---- per-lane LDS read addresses (stage 0; stage 1 adds the section's stage size) ----
  const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)alds;
  const int qrow = 32 * qb + m;
  uint32_t aB[8], aV[4], aK[2];
#pragma unroll
  for (int u = 0; u < 2; ++u)            // key half u, accumulator register group g
#pragma unroll
    for (int g = 0; g < 4; ++g)
      aB[4 * u + g] = base + TS_BIAS + 256 * qrow + 16 * ((8 * u + 2 * g + h) ^ (qrow & 15));
#pragma unroll
  for (int c = 0; c < 4; ++c)            // c = 2 u + s: chunk 2c + h of a 64-key V^T row
    aV[c] = base + TS_V + 4096 * row + 128 * m + 16 * ((2 * c + h) ^ swz8(m));
  const int ksw = swz4(m);
#pragma unroll
  for (int s = 0; s < 2; ++s) aK[s] = base + TS_K + 4096 * row + 64 * m + 16 * ((2 * s + h) ^ ksw);
  uint32_t aM = base + TS_MASK + 128 * row + 2 * m;
  // opaque to the optimizer: each read is then one address register + an immediate offset
#pragma unroll
  for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(aB[i]));
#pragma unroll
  for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(aV[i]));
  asm volatile("" : "+v"(aK[0]), "+v"(aK[1]), "+v"(aM));

  issue(0, h0, 0);   // the first stage's DMA overlaps the scan below
  // rows whose valid keys are all masked (wave-uniform)
  bool live_l = false;
  {
    const op_t* mr = mask16 + ((long)b * N + ip) * N;
    for (int k = lane; k < n_valid; k += 64) live_l |= (float)mr[k] != -INFINITY;
  }
  const bool live = __ballot(live_l) != 0;

  const uint32_t ONE = half_bits((op_t)1.f);
  const uint32_t lo_half = h ? 0u : ~0u;   // keeps a value in lanes 0-31, zero in 32-63
  // the rank-1 operands are 4-register tuples whose words 1..3 stay zero: only word 0 changes
  // ([-m, 1] of the block's reference in fb, [1, mask] of the key half in ra), half 1 of the
  // wave holds zero
  u32x4 fb = {0u, 0u, 0u, 0u}, ra = {0u, 0u, 0u, 0u};
  auto set_fb = [&](float mv) PF_INLINE {
    fb[0] = h ? 0u : (half_bits((op_t)(-mv)) | ONE << 16);
    asm volatile("" : "+v"(fb));
  };

  const int jq0 = jw0 + 32 * qb;   // first query of this wave's block; blocks past N idle
  const bool qvalid = jq0 < N;
  opx8 qf[2], qn[2];   // this head's Q fragments, the next head's (loaded a step ahead)
  f32x16 o;
  float mh, lsum;
  uint64_t mset;   // lane mask: the queries (lanes) that have a reference maximum
  auto q_fetch = [&](int hd) PF_INLINE {
    const int jq = min(jq0, N - 32);
    const op_t* qptr = Q + ((((long)b * N + ip) * H + hd) * N + jq + m) * D + 8 * h;
#pragma unroll
    for (int s = 0; s < 2; ++s) qn[s] = ld_x8(qptr + 16 * s);
  };
  auto head_start = [&]() PF_INLINE {
    o = zero16();
    lsum = 0.f;
    mh = 0.f;
    mset = 0;
    set_fb(0.f);
  };
  // P = exp2(S') packed into the two P.V operands; returns the lane's row sum
  auto exp_pack = [&](const f32x16& sc, u32x4 (&pf)[2]) PF_INLINE {
    float ls[2] = {0.f, 0.f};   // two partial sums: half as long a v_dot2 chain
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int t2 = 0; t2 < 8; t2 += 2) {
        opx2 pk;
        pk[0] = (op_t)exp2_fast(sc[8 * ks + t2]);
        pk[1] = (op_t)exp2_fast(sc[8 * ks + t2 + 1]);
        ls[ks] = dot2_ones(pk, ls[ks]);
        pf[ks][t2 >> 1] = __builtin_bit_cast(uint32_t, pk);
      }
    return ls[0] + ls[1];
  };
  // One step (stage STG) of a live row: the block's two 32x32 tiles (key halves u) one after the
  // other: scores (bias as the accumulator start, K.Q^T, the mask / reference fold), the softmax
  // against the current reference, one check, and the two P.V MFMAs.  When the check fails (no
  // reference yet -- every head's first tile -- or a tile row sum above LSTEP_MAX) the reference
  // moves to the tile's maximum first; the next tile's scores already use the new reference.
  auto step2 = [&](auto stg) PF_INLINE {
    constexpr int STG = decltype(stg)::value;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      // every lane reads its key's mask entry (an in-bounds address for all lanes; half 1
      // discards it) together with the tile's other reads: a read inside an h == 0 branch
      // would get an LDS wait of its own ahead of them
      const uint32_t mk = lds_rd16(aM + STG * TM_STAGE + 64 * u);
      f32x16 sc;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 bv = lds_rd4f(aB[4 * u + g] + STG * TB_STAGE);
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[4 * g + e] = bv[e];
      }
      // every fragment of the tile is read before the first MFMA (one LDS round trip, and the
      // P.V operands are not behind the rescale branch)
      const opx8 k0 = lds_rd8(aK[0] + STG * TK_STAGE + 2048 * u), k1 = lds_rd8(aK[1] + STG * TK_STAGE + 2048 * u);
      const opx8 v0 = lds_rd8(aV[2 * u] + STG * TV_STAGE), v1 = lds_rd8(aV[2 * u + 1] + STG * TV_STAGE);
      // raised issue priority while the wave issues its score MFMAs, so a wave that has its
      // operands gets the MFMA pipe ahead of the others' exponentials (2-3 % at N = 512)
      __builtin_amdgcn_s_setprio(2);
      sc = mfma32(k0, qf[0], sc);
      sc = mfma32(k1, qf[1], sc);
      ra[0] = (ONE | mk << 16) & lo_half;
      asm volatile("" : "+v"(ra));
      sc = mfma32(as_x8(ra), as_x8(fb), sc);
      __builtin_amdgcn_s_setprio(0);
      u32x4 pf[2];
      float l = exp_pack(sc, pf);
      // the lane masks come straight from v_cmp (a bool ballot would materialize and re-test
      // each lane's predicate); every lane is active here (a live row's valid query block)
      if ((__builtin_amdgcn_fcmpf(l, LSTEP_MAX, 2 /* ordered > */) | ~mset) != 0) {
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[r]);
        mx = xor32_max(mx);
        const bool ms = (mset >> lane) & 1;
        const float d = ms ? (mx > RESCALE_SLACK ? mx : 0.f) : (mx == -INFINITY ? 0.f : mx);
        const float mnew = (float)(op_t)(mh + d);
        const float dsub = mnew - mh;
        const float alpha = ms ? exp2_fast(-dsub) : 1.f;
        lsum *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) o[r] *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[r] -= dsub;
        l = exp_pack(sc, pf);
        mset |= __builtin_amdgcn_fcmpf(mx, -INFINITY, 14 /* unordered or != */);
        mh = mnew;
        set_fb(mnew);
      }
      lsum += l;
      o = mfma32(v0, as_x8(pf[0]), o);
      o = mfma32(v1, as_x8(pf[1]), o);
    }
  };
  auto finalize = [&](int hd) PF_INLINE {
    if (!qvalid) return;
    const float inv = rcp_fast(xor32_sum(lsum));
    const int j = jq0 + m;
    const long rowbase = ((long)b * N + ip) * H;
    if (OUT_F32) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = o[4 * g + e] * inv;
        *reinterpret_cast<f32x4*>(O32 + ((rowbase + hd) * N + j) * D + 8 * g + 4 * h) = v;
      }
    } else {
      store_runs16(O16 + (((long)b * N + ip) * N + j) * C + 32 * hd, o, inv, h);   // 16-byte runs
    }
  };

  // Step loop: T steps (T = 4 N / 64, even), one barrier each (the loop-top wait + barrier),
  // the DMA of the next step into the other stage; during a head's last step the next head's
  // Q is loaded (it lands by the next loop-top wait).  The barrier also tells every wave that
  // the other stage (read in the previous step) is free.
  int kbi = 0, hd = h0;  // step it = (hd - h0) * nKB + kbi
  if (qvalid && live) q_fetch(h0);
  auto one_step = [&](auto stg, int it) PF_INLINE {
    constexpr int STG = decltype(stg)::value;
    __builtin_amdgcn_s_waitcnt(vmcnt_le(0));   // this wave's part of stage STG (and Q) landed ...
    __builtin_amdgcn_s_barrier();              // ... for every wave; stage STG ^ 1 is free
    asm volatile("" ::: "memory");
    if (it + 1 < T) {
      const bool wrap = kbi + 1 == nKB;
      issue(STG ^ 1, wrap ? hd + 1 : hd, wrap ? 0 : 64 * (kbi + 1));
    }
    if (qvalid && live) {
      if (kbi == 0) {
        head_start();
        qf[0] = qn[0];
        qf[1] = qn[1];
      }
      if (kbi == nKB - 1 && hd + 1 < h0 + nh) q_fetch(hd + 1);   // lands by the next step's wait
      step2(stg);
      if (kbi == nKB - 1) finalize(hd);
    }
    if (++kbi == nKB) {
      kbi = 0;
      ++hd;
    }
  };
  for (int it = 0; it < T; it += 2) {
    one_step(ic<0>{}, it);
    one_step(ic<1>{}, it + 1);
  }

  // A dead row (every valid key masked): the reference's logits all round to -1e9, so each
  // query's output is the plain mean of v over the n_valid keys, the same for every query of
  // the row.  The row's four query-block waves split its four heads: wave qb sums head qb's
  // V^T (keys stored at perm16 positions) for d = m, the two lane halves taking alternate
  // 16-byte chunks (8 loads in flight, v_dot2 pair sums, keys past n_valid zeroed by
  // selects), and the means meet in LDS.  Every wave takes part in both barriers.
  static_assert(H == TA_WAVES / 4, "one head per query-block wave of a row");
  __syncthreads();   // the last step's stage reads are done before the LDS is reused
  float* smean = reinterpret_cast<float*>(alds);   // [4 rows][H][D]
  if (!live && qb < nh) {
    const int hd2 = h0 + qb;
    const bool all_valid = n_valid >= N;   // wave-uniform
    const op_t* vrow = Vt + ((((long)b * N + ip) * H + hd2) * D + m) * (long)N;
    float acc = 0.f;
    for (int p0 = 8 * h; p0 < N; p0 += 16 * 8) {   // 8 stored keys per 16-byte load
      opx8 v8[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v8[u] = p0 + 16 * u < N ? ld_x8(vrow + p0 + 16 * u) : zero_x8();
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          opx2 pr = {v8[u][e], v8[u][e + 1]};
          if (!all_valid) {
            pr[0] = perm16(p0 + 16 * u + e) < n_valid ? pr[0] : (op_t)0.f;
            pr[1] = perm16(p0 + 16 * u + e + 1) < n_valid ? pr[1] : (op_t)0.f;
          }
          acc = dot2_ones(pr, acc);
        }
    }
    const float mean = xor32_sum(acc) / (float)n_valid;   // lanes m and m + 32 both hold d = m
    if (h == 0) smean[(row * H + hd2) * D + m] = mean;
  }
  __syncthreads();
  if (!live && qvalid) {
    const int j = jq0 + m;
    for (int hd2 = h0; hd2 < h0 + nh; ++hd2) {
      const float* mrow = smean + (row * H + hd2) * D;
      if (OUT_F32) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          *reinterpret_cast<f32x4*>(O32 + ((((long)b * N + ip) * H + hd2) * N + j) * D + 16 * h + 4 * q4) =
              *reinterpret_cast<const f32x4*>(mrow + 16 * h + 4 * q4);
      } else {
#pragma unroll
        for (int q8 = 0; q8 < 2; ++q8) {
          opx8 v;
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = (op_t)mrow[16 * h + 8 * q8 + e];
          st_x8(O16 + (((long)b * N + ip) * N + j) * C + 32 * hd2 + 16 * h + 8 * q8, v);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Output projection: z[pair(i, j)] (+)= linear_o(O[i, j] * sigmoid(linear_g(LN(z[pair])))).
// Persistent: one workgroup (8 waves) per CU keeps W_g and W_o in LDS (op_t as given, so rounded
// once) with the LayerNorm's beta folded into fp32 gate offsets -log2(e) W_g beta (gamma scales
// the normalized z before its rounding to op_t); each wave walks tiles of 32 frame positions
// (ip, j0 .. j0+31).  Everything is in the output-aligned layout (pf_common.h): the gate comes
// out of D[channel][position] = W_g . LN(z) in the same channel order as the O values the lane
// loads, o * sigmoid(g) is directly the B operand of D[out][position] = W_o . (o * g), and the
// residual is the z the lane loaded.  Weight rows are 4 op_t longer than their width, so the
// 8-byte fragment reads of 32 rows fall on distinct banks.
// FAST (the fast mode's block-fp8 points): the gate's offsets are W_g beta itself, and g
// (per head: one 32-channel block, a lane pair's 16 + 16 registers) and the projection's
// output (per 32 output channels) are quantize-dequantized before the sigmoid and before
// the residual.
// ---------------------------------------------------------------------------------
constexpr int TAO_WAVES = 8;
// LDS: the gate offsets [C] and gamma [CC] (fp32, first: small immediate offsets), then
// W_g [C][CC + 4] and W_o [CC][C + 4] op_t, then (HILO) their residuals in the same layout
template <int CC, bool HILO = false>
constexpr size_t tao_lds() {
  return (C + CC) * sizeof(float) + (HILO ? 2 : 1) * ((size_t)C * (CC + 4) + (size_t)CC * (C + 4)) * sizeof(op_t);
}

// resid: 0 -> out = update; 1 -> out = z_in + update (out may alias z_in); 2 -> out += update
// HILO: W_g and W_o come with their residuals wg_lo = W_g - W_g16, wo_lo = W_o - W_o16 (rounded
// to op_t), and both products run on hi + lo (two MFMAs per fragment): weights good to ~2^-22
// of their size instead of the 2^-12 of one 16-bit rounding.  The gate's offsets use hi + lo.
template <int CC, bool FAST, bool HILO = false>
__global__ __launch_bounds__(64 * TAO_WAVES, 1) void ta_out_kernel(
    const op_t* __restrict__ O, const float* z_in, float* out, const float* __restrict__ lnw,
    const float* __restrict__ lnb, const op_t* __restrict__ wg, const op_t* __restrict__ wo,
    const op_t* __restrict__ wg_lo, const op_t* __restrict__ wo_lo,
    int B, int N, int ending, int resid, float eps) {
  constexpr int LWG = CC + 4, LWO = C + 4, KS = CC / 16;
  extern __shared__ __attribute__((aligned(16))) op_t tlds[];
  float* cgate = reinterpret_cast<float*>(tlds);
  float* gam = cgate + C;
  op_t* sWg = tlds + 2 * (C + CC);
  op_t* sWo = sWg + C * LWG;
  op_t* sWgl = sWo + CC * LWO;   // HILO only
  op_t* sWol = sWgl + C * LWG;
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, m = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  {   // weights -> LDS: every chunk of this thread loaded before the first store
    constexpr int NT = 64 * TAO_WAVES;
    static_assert(CC <= NT, "gamma: one value per thread");
    opx8 vg[stage_per<NT, C, CC>()], vo[stage_per<NT, CC, C>()];
    stage_load<NT, C, CC>(wg, vg);
    stage_load<NT, CC, C>(wo, vo);
    const float gv = tid < CC ? lnw[tid] : 0.f;
    if constexpr (HILO) {
      opx8 vgl[stage_per<NT, C, CC>()], vol[stage_per<NT, CC, C>()];
      stage_load<NT, C, CC>(wg_lo, vgl);
      stage_load<NT, CC, C>(wo_lo, vol);
      stage_store<NT, C, CC>(sWgl, LWG, vgl);
      stage_store<NT, CC, C>(sWol, LWO, vol);
    }
    stage_store<NT, C, CC>(sWg, LWG, vg);
    stage_store<NT, CC, C>(sWo, LWO, vo);
    if (tid < CC) gam[tid] = gv;
  }
  __syncthreads();
  for (int row = tid; row < C; row += 64 * TAO_WAVES) {   // gate offsets -log2(e) W_g beta (weights from LDS)
    const op_t* w = sWg + row * LWG;
    const op_t* wl = sWgl + row * LWG;
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < CC; c += 8) {
      const opx4 wa = ld_x4(w + c), wb = ld_x4(w + c + 4);
      const opx8 w8 = {wa[0], wa[1], wa[2], wa[3], wb[0], wb[1], wb[2], wb[3]};
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += (float)w8[e] * lnb[c + e];
      if constexpr (HILO) {
        const opx4 la = ld_x4(wl + c), lb = ld_x4(wl + c + 4);
        const opx8 l8 = {la[0], la[1], la[2], la[3], lb[0], lb[1], lb[2], lb[3]};
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += (float)l8[e] * lnb[c + e];
      }
    }
    cgate[row] = FAST ? acc : -LOG2E * acc;
  }
  __syncthreads();
  const uint32_t ntiles = (uint32_t)B * N * N / 32;
  const uint32_t stride = gridDim.x * TAO_WAVES;
  uint32_t t = blockIdx.x * TAO_WAVES + wid;
  for (; t < ntiles; t += stride) {
    asm volatile("" ::: "memory");   // the gate offsets are re-read from LDS each tile, not pinned in VGPRs
    const PosTile pt = pos_tile(t, N);
    const int b = pt.b, ip = pt.r, j = pt.c0 + m;
    const long zp = ending ? ((long)b * N + j) * N + ip : ((long)b * N + ip) * N + j;
    opx8 xf[KS];
    float zr[CC / 2];
    load_row_oa<CC>(z_in + zp * CC, h, zr);
    ln_oa_gamma_to_frag<CC>(zr, h, gam, eps, xf);
    // o * sigmoid(g) as the B operand of the output projection (k order = output-aligned)
    opx4 ov4[C / 8];   // O values (C = H * D channels): oa_channel(q, h) + 0..3 of position 32 t + m
#pragma unroll
    for (int q = 0; q < C / 8; ++q) ov4[q] = ld_x4(O + (32l * t + m) * C + oa_channel(q, h));
    opx8 og[8];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const op_t* wrow = &sWg[(32 * cb + m) * LWG];
      f32x16 g = zero16();
#pragma unroll
      for (int s = 0; s < KS; ++s) g = mfma32(wfrag_oa(wrow, s, h), xf[s], g);   // D[channel][position]
      if constexpr (HILO) {
        const op_t* wlrow = &sWgl[(32 * cb + m) * LWG];
#pragma unroll
        for (int s = 0; s < KS; ++s) g = mfma32(wfrag_oa(wlrow, s, h), xf[s], g);
      }
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
        const int q = 4 * cb + gg;            // chunk: channels oa_channel(q, h) + 0..3
        const opx4 ov = ov4[q];
        const f32x4 cg = *reinterpret_cast<const f32x4*>(cgate + oa_channel(q, h));
        if constexpr (FAST) {
#pragma unroll
          for (int e = 0; e < 4; ++e) g[4 * gg + e] += cg[e];
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            og[q >> 1][4 * (q & 1) + e] =
                (op_t)((float)ov[e] * rcp_fast(1.f + exp2_fast(fmaf(g[4 * gg + e], -LOG2E, cg[e]))));
        }
      }
      if constexpr (FAST) {
        mx_fake_quant16(g);
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
          const int q = 4 * cb + gg;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            og[q >> 1][4 * (q & 1) + e] =
                (op_t)((float)ov4[q][e] * rcp_fast(1.f + exp2_fast(-LOG2E * g[4 * gg + e])));
        }
      }
    }
#pragma unroll
    for (int ob = 0; ob < CC / 32; ++ob) {
      const op_t* wrow = &sWo[(32 * ob + m) * LWO];
      f32x16 acc = zero16();
#pragma unroll
      for (int s = 0; s < 8; ++s) acc = mfma32(wfrag_oa(wrow, s, h), og[s], acc);   // D[out][position]
      if constexpr (HILO) {
        const op_t* wlrow = &sWol[(32 * ob + m) * LWO];
#pragma unroll
        for (int s = 0; s < 8; ++s) acc = mfma32(wfrag_oa(wlrow, s, h), og[s], acc);
      }
      if constexpr (FAST) mx_fake_quant16(acc);
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
        const int q = 4 * ob + gg;
        float* dst = out + zp * CC + oa_channel(q, h);
        f32x4 v;
        if (resid == 1) v = f32x4{zr[4 * q], zr[4 * q + 1], zr[4 * q + 2], zr[4 * q + 3]};
        if (resid == 2) v = *reinterpret_cast<const f32x4*>(dst);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = resid == 0 ? acc[4 * gg + e] : v[e] + acc[4 * gg + e];
        *reinterpret_cast<f32x4*>(dst) = v;
      }
    }
  }
}

// Layout conversion for the standalone attention core (fp32 API tensors -> kernel layout).
// A workgroup takes 64 keys of one (b, i, h) sequence: q / k as 8-value runs per thread
// (coalesced 32-byte loads, 16-byte stores), v through an LDS transpose so that every V^T row
// (d) leaves as 16-byte runs of 8 stored keys.
constexpr int PREP_KB = 64;
__global__ __launch_bounds__(256) void ta_prep_qkv_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                          const float* __restrict__ v, float qs,
                                                          op_t* __restrict__ Q, op_t* __restrict__ K,
                                                          op_t* __restrict__ Vt, int N) {
  __shared__ op_t sV[D][PREP_KB + 8];   // [d][key within the block], rows 16 bytes longer
  const int nb = N / PREP_KB;
  const long r = blockIdx.x / nb;                       // sequence (b, i, h)
  const int j0 = (int)(blockIdx.x - r * nb) * PREP_KB;
  const int tid = threadIdx.x, jl = tid >> 2, d0 = (tid & 3) * 8;
  const long e = (r * N + j0 + jl) * D + d0;           // element (key j0 + jl, d0) of q / k / v
  const f32x4 q0 = *reinterpret_cast<const f32x4*>(q + e), q1 = *reinterpret_cast<const f32x4*>(q + e + 4);
  const f32x4 k0 = *reinterpret_cast<const f32x4*>(k + e), k1 = *reinterpret_cast<const f32x4*>(k + e + 4);
  const f32x4 v0 = *reinterpret_cast<const f32x4*>(v + e), v1 = *reinterpret_cast<const f32x4*>(v + e + 4);
  opx8 oq, ok;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    oq[u] = (op_t)(q0[u] * qs);
    oq[4 + u] = (op_t)(q1[u] * qs);
    ok[u] = (op_t)k0[u];
    ok[4 + u] = (op_t)k1[u];
    sV[d0 + u][jl] = (op_t)v0[u];
    sV[d0 + 4 + u][jl] = (op_t)v1[u];
  }
  st_x8(Q + e, oq);
  st_x8(K + e, ok);
  __syncthreads();
  // V^T row d = tid / 8, stored positions 8 c .. 8 c + 7 hold keys perm16(8 c + i) (perm16 is
  // its own inverse and keeps every 16-key group in place)
  const int d = tid >> 3, c = tid & 7;
  opx8 ov;
#pragma unroll
  for (int i = 0; i < 8; ++i) ov[i] = sV[d][perm16(8 * c + i)];
  st_x8(Vt + (r * D + d) * N + j0 + 8 * c, ov);
}

__global__ void ta_prep_bias_kernel(const float* __restrict__ bias, const float* __restrict__ mask,
                                    float* __restrict__ bias32, op_t* __restrict__ mask16,
                                    long nbias, long nmask, int N, int n_valid) {
  for (long e = (long)blockIdx.x * blockDim.x + threadIdx.x; e < nbias; e += (long)gridDim.x * blockDim.x) {
    bias32[e] = bias[e] * LOG2E;
    if (e < nmask) mask16[e] = mask_term((int)(e % N) >= n_valid, mask ? mask[e] : 1.f);
  }
}

struct TaBuffers {
  op_t *Q, *K, *Vt, *O;
  float* bias32;
  op_t* mask16;
  float* stats;   // the mean-correction partials
};

// Workspace: Q, K, V^T, O (op_t, [B][N][H][N][D] each), the fp32 bias [B][H][N][N], the op_t
// mask term [B][N][N].
size_t ta_buffers_size(int B, int N) {
  const size_t e = (size_t)B * N * H * N * D;
  const size_t bytes = 4 * e * sizeof(op_t) + (size_t)B * H * N * N * sizeof(float) + (size_t)B * N * N * sizeof(op_t);
  return (bytes + 15) / 16 * 16 + PS_PARTIAL_FLOATS * sizeof(float);   // + the mean-correction partials
}

TaBuffers ta_buffers(void* ws, int B, int N) {
  const size_t e = (size_t)B * N * H * N * D;
  TaBuffers t;
  t.Q = (op_t*)ws;
  t.K = t.Q + e;
  t.Vt = t.K + e;
  t.O = t.Vt + e;
  t.bias32 = reinterpret_cast<float*>(t.O + e);
  t.mask16 = reinterpret_cast<op_t*>(t.bias32 + (size_t)B * H * N * N);
  const size_t used = (size_t)((char*)(t.mask16 + (size_t)B * N * N) - (char*)ws);
  t.stats = reinterpret_cast<float*>((char*)ws + (used + 15) / 16 * 16);
  return t;
}

template <bool OUT_F32>
int launch_attn(const TaBuffers& t, float* o32, int B, int N, int n_valid, hipStream_t st) {
  if (const int rc = pf_reserve_lds((const void*)ta_attn_kernel<OUT_F32>, TA_LDS, "ta_attn_kernel")) return rc;
  const int total = B * (N / 4) * ((N + 127) / 128);
  // the blocks of a last round (all of them when the launch is one round or less) that would fill
  // at most half of the CUs run split over 2 or 4 workgroups, H / split heads each: the largest
  // split whose workgroups still fit on the chip
  const int cus = device_cus();
  const int rest = cus <= 0 ? 0 : total > cus ? total % cus : total;
  // (the kernel takes its H / split * N / 64 steps in pairs, one per ring stage: a single-head
  // split needs an even N / 64)
  int split = 1;
  while (split < 4 && rest > 0 && 2 * split * rest <= cus && !(split == 2 && (N / 64) % 2)) split *= 2;
  const int full = split > 1 ? total - rest : total;
  static_assert(H % 4 == 0, "head splits of 2 and 4");
  pf_attend_mark(st, 0);
  ta_attn_kernel<OUT_F32><<<full + split * (total - full), 64 * TA_WAVES, TA_LDS, st>>>(
      t.Q, t.K, t.Vt, t.bias32, t.mask16, t.O, o32, N, n_valid, total, full, split > 1 ? split : 2);
  PF_CHECK_LAUNCH("ta_attn_kernel");
  pf_attend_mark(st, 1);
  return PF_OK;
}

// e4m3 bytes q [rows][K] with E8M0 scale bytes s [rows][K / 32] (pf_quantize_mx8) -> op_t
// values e4m3 * 2^(s - 127), exact in op_t for the weights' range; n % 4 == 0, K % 32 == 0.
// A scale byte 0 (an all-zero block) gives zeros.
__global__ void mx8_dequant_kernel(const uint8_t* __restrict__ q, const uint8_t* __restrict__ s,
                                   op_t* __restrict__ out, long n, int K) {
  for (long e = 4 * ((long)blockIdx.x * blockDim.x + threadIdx.x); e < n; e += 4l * gridDim.x * blockDim.x) {
    const int word = *reinterpret_cast<const int*>(q + e);
    const long row = e / K;
    const float X = __uint_as_float((uint32_t)s[row * (K / 32) + (e - row * K) / 32] << 23);
    const auto lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word, X, false);
    const auto hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word, X, true);
    st_x4(out + e, opx4{(op_t)lo[0], (op_t)lo[1], (op_t)hi[0], (op_t)hi[1]});
  }
}

// W_q, W_k, W_v, W_g as the kernels read them (op_t [C][CC]); the residuals of W_g and W_o
// (op_t, or null).
struct TaWeights { const op_t *q, *k, *v, *g, *g_lo = nullptr, *o_lo = nullptr; };

// The mean correction of ta_proj's weights for a 16-bit call with the exact offsets and the
// four folded-weight residuals, one batch element, c_z = 128 (else the plain W16 beta offsets).
template <int CC, bool FAST>
TaMeanFix ta_mean_fix(const pf_triatt_args* a, const TaBuffers& t, hipStream_t st, int* rc) {
  TaMeanFix mf{nullptr, {nullptr, nullptr, nullptr, nullptr}, nullptr};
  *rc = PF_OK;
  if (FAST || CC != PS_C || !a->in_offsets) return mf;
  mf.offb = a->in_offsets;
  if (a->B == 1 && a->w_q_lo && a->w_k_lo && a->w_v_lo && a->w_bias_lo) {
    mf.lo[0] = (const op_t*)a->w_q_lo; mf.lo[1] = (const op_t*)a->w_k_lo;
    mf.lo[2] = (const op_t*)a->w_v_lo; mf.lo[3] = (const op_t*)a->w_bias_lo;
    mf.stats = t.stats;
    pair_stats_kernel<<<PS_WG, 64 * PS_WAVES, 0, st>>>(a->z_in, a->N, a->eps, t.stats);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) *rc = pf_fail(PF_E_LAUNCH, "pair_stats_kernel launch failed: %s", hipGetErrorString(e));
  }
  return mf;
}

template <int CC, bool FAST>
int triatt_run(const pf_triatt_args* a, const TaWeights& w) {
  hipStream_t st = (hipStream_t)a->stream;
  const int B = a->B, N = a->N;
  const int n_valid = a->n_valid ? a->n_valid : N;
  TaBuffers t = ta_buffers(a->workspace, B, N);
  const float qscale = LOG2E / sqrtf((float)D);
  const long positions = (long)B * N * N;
  const int cus = device_cus();
  if (cus <= 0) return pf_fail(PF_E_LAUNCH, "pf_triatt_fwd: cannot query the device");
  int mrc = PF_OK;
  const TaMeanFix mf = ta_mean_fix<CC, FAST>(a, t, st, &mrc);
  if (mrc) return mrc;
  {
    const void* fn = (const void*)ta_proj_kernel<CC, FAST>;
    if (const int rc = pf_reserve_lds(fn, tap_lds<CC, FAST>(), "ta_proj_kernel")) return rc;
    const int grid = (int)min((long)cus, (positions / 32 + TAP_WAVES - 1) / TAP_WAVES);
    ta_proj_kernel<CC, FAST><<<grid, 64 * TAP_WAVES, tap_lds<CC, FAST>(), st>>>(
        a->z_in, a->pair_mask, a->ln_w, a->ln_b, w.q, w.k, w.v, (const op_t*)a->w_bias, t.Q, t.K, t.Vt, t.bias32,
        t.mask16, B, N, n_valid, a->ending, qscale, a->eps, mf);
    PF_CHECK_LAUNCH("ta_proj_kernel");
  }
  int rc = launch_attn<false>(t, nullptr, B, N, n_valid, st);
  if (rc) return rc;
  {
    const int grid = (int)min((long)cus, (positions / 32 + TAO_WAVES - 1) / TAO_WAVES);
    const int resid = !a->accumulate ? 0 : (a->out == a->z_in ? 1 : 2);
    bool hilo = false;
    if constexpr (!FAST && CC == 128) {   // the residual weights exist for the 16-bit c_z = 128 path
      if (w.g_lo && w.o_lo) {
        hilo = true;
        const void* fn = (const void*)ta_out_kernel<CC, FAST, true>;
        if (const int rc = pf_reserve_lds(fn, tao_lds<CC, true>(), "ta_out_kernel")) return rc;
        ta_out_kernel<CC, FAST, true><<<grid, 64 * TAO_WAVES, tao_lds<CC, true>(), st>>>(
            t.O, a->z_in, a->out, a->ln_w, a->ln_b, w.g, (const op_t*)a->w_o, w.g_lo, w.o_lo, B, N, a->ending, resid,
            a->eps);
      }
    }
    if (!hilo) {
      const void* fn = (const void*)ta_out_kernel<CC, FAST>;
      if (const int rc = pf_reserve_lds(fn, tao_lds<CC>(), "ta_out_kernel")) return rc;
      ta_out_kernel<CC, FAST><<<grid, 64 * TAO_WAVES, tao_lds<CC>(), st>>>(
          t.O, a->z_in, a->out, a->ln_w, a->ln_b, w.g, (const op_t*)a->w_o, nullptr, nullptr, B, N, a->ending,
          resid, a->eps);
    }
    PF_CHECK_LAUNCH("ta_out_kernel");
  }
  return PF_OK;
}

// The attention kernel addresses a batch's bias ([H][N][N] fp32) through one raw buffer
// resource, whose range is below 2^31 bytes.
bool ta_shape_ok(int N) { return (long)H * N * N * 4 < (1l << 31); }

}  // namespace

// ---------------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------------
extern "C" size_t pf_triatt_workspace_size(int B, int N, int C_, int H_, int D_) {
  if (B <= 0 || N <= 0 || (C_ != 128 && C_ != 64) || H_ != H || D_ != D) return 0;
  return ta_buffers_size(B, N);
}

extern "C" int pf_triatt_fwd(const pf_triatt_args* a) {
  if (!a) return pf_fail(PF_E_INVALID, "pf_triatt_fwd: null args");
  if ((a->C != 128 && a->C != 64) || a->H != H || a->D != D)
    return pf_fail(PF_E_INVALID, "pf_triatt_fwd: only C = 128 or 64, H=4, D=32 supported (got C=%d H=%d D=%d)",
                   a->C, a->H, a->D);
  if (a->B <= 0 || a->N <= 0 || a->N % 64)
    return pf_fail(PF_E_INVALID, "pf_triatt_fwd: need B > 0 and N a positive multiple of 64 (B=%d N=%d)", a->B, a->N);
  if ((unsigned long long)a->B * a->N * a->N >= (1ull << 32) || !ta_shape_ok(a->N))
    return pf_fail(PF_E_INVALID, "pf_triatt_fwd: need B * N * N < 2^32 and N <= 11584 (B=%d N=%d)", a->B, a->N);
  if (!a->z_in || !a->out || !a->ln_w || !a->ln_b || !a->w_bias || !a->w_q || !a->w_k ||
      !a->w_v || !a->w_g || !a->w_o || !a->workspace)
    return pf_fail(PF_E_INVALID, "pf_triatt_fwd: null pointer argument");
  const size_t need = ta_buffers_size(a->B, a->N);
  if (a->workspace_bytes < need)
    return pf_fail(PF_E_INVALID, "pf_triatt_fwd: workspace too small (%zu < %zu bytes)", a->workspace_bytes, need);
  if (a->n_valid < 0 || a->n_valid > a->N)
    return pf_fail(PF_E_INVALID, "pf_triatt_fwd: n_valid %d outside [0, N=%d]", a->n_valid, a->N);
  if ((a->w_g_lo != nullptr) != (a->w_o_lo != nullptr) || (a->w_g_lo && a->C != 128))
    return pf_fail(PF_E_INVALID, "pf_triatt_fwd: give both weight residuals (w_g_lo, w_o_lo) or neither, C = 128 only");
  {
    const bool any_lo = a->w_q_lo || a->w_k_lo || a->w_v_lo || a->w_bias_lo;
    if ((a->in_offsets || any_lo) && a->C != 128)
      return pf_fail(PF_E_INVALID, "pf_triatt_fwd: exact offsets and the mean correction need C = 128");
    if (any_lo && !(a->in_offsets && a->w_q_lo && a->w_k_lo && a->w_v_lo && a->w_bias_lo))
      return pf_fail(PF_E_INVALID, "pf_triatt_fwd: the mean correction needs in_offsets and all four residuals "
                                   "(w_q_lo, w_k_lo, w_v_lo, w_bias_lo)");
  }
  const TaWeights w = {(const op_t*)a->w_q, (const op_t*)a->w_k, (const op_t*)a->w_v, (const op_t*)a->w_g,
                       (const op_t*)a->w_g_lo, (const op_t*)a->w_o_lo};
  return a->C == 128 ? triatt_run<128, false>(a, w) : triatt_run<64, false>(a, w);
}

// Fast mode: the 16-bit workspace, then W_q, W_k, W_v, W_g dequantized to op_t [4][C][C].
extern "C" size_t pf_triatt_mx8_workspace_size(int B, int N, int C_, int H_, int D_) {
  if (B <= 0 || N <= 0 || C_ != 128 || H_ != H || D_ != D) return 0;
  return ta_buffers_size(B, N) + 4 * (size_t)C * C * sizeof(op_t);
}

extern "C" int pf_triatt_mx8_fwd(const pf_triatt_mx8_args* m) {
  if (!m) return pf_fail(PF_E_INVALID, "pf_triatt_mx8_fwd: null args");
  if (m->C != 128 || m->H != H || m->D != D)
    return pf_fail(PF_E_INVALID, "pf_triatt_mx8_fwd: only C = 128, H=4, D=32 supported (got C=%d H=%d D=%d)", m->C,
                   m->H, m->D);
  if (m->B <= 0 || m->N <= 0 || m->N % 64)
    return pf_fail(PF_E_INVALID, "pf_triatt_mx8_fwd: need B > 0 and N a positive multiple of 64 (B=%d N=%d)", m->B,
                   m->N);
  if ((unsigned long long)m->B * m->N * m->N >= (1ull << 32) || !ta_shape_ok(m->N))
    return pf_fail(PF_E_INVALID, "pf_triatt_mx8_fwd: need B * N * N < 2^32 and N <= 11584 (B=%d N=%d)", m->B, m->N);
  if (!m->z_in || !m->out || !m->ln_w || !m->ln_b || !m->w_bias || !m->w_q_q || !m->w_q_s || !m->w_k_q ||
      !m->w_k_s || !m->w_v_q || !m->w_v_s || !m->w_g_q || !m->w_g_s || !m->w_o || !m->workspace)
    return pf_fail(PF_E_INVALID, "pf_triatt_mx8_fwd: null pointer argument");
  const size_t need = pf_triatt_mx8_workspace_size(m->B, m->N, m->C, m->H, m->D);
  if (m->workspace_bytes < need)
    return pf_fail(PF_E_INVALID, "pf_triatt_mx8_fwd: workspace too small (%zu < %zu bytes)", m->workspace_bytes, need);
  if (m->n_valid < 0 || m->n_valid > m->N)
    return pf_fail(PF_E_INVALID, "pf_triatt_mx8_fwd: n_valid %d outside [0, N=%d]", m->n_valid, m->N);
  hipStream_t st = (hipStream_t)m->stream;
  op_t* wd = reinterpret_cast<op_t*>((char*)m->workspace + ta_buffers_size(m->B, m->N));
  const void* src[4][2] = {{m->w_q_q, m->w_q_s}, {m->w_k_q, m->w_k_s}, {m->w_v_q, m->w_v_s}, {m->w_g_q, m->w_g_s}};
  for (int i = 0; i < 4; ++i) {
    mx8_dequant_kernel<<<16, 256, 0, st>>>((const uint8_t*)src[i][0], (const uint8_t*)src[i][1], wd + i * C * C,
                                          (long)C * C, C);
    PF_CHECK_LAUNCH("mx8_dequant_kernel");
  }
  pf_triatt_args a = {};
  a.B = m->B; a.N = m->N; a.C = m->C; a.H = m->H; a.D = m->D;
  a.ending = m->ending; a.accumulate = m->accumulate; a.n_valid = m->n_valid; a.eps = m->eps;
  a.z_in = m->z_in; a.out = m->out; a.pair_mask = m->pair_mask; a.ln_w = m->ln_w; a.ln_b = m->ln_b;
  a.w_bias = m->w_bias; a.w_o = m->w_o;
  a.workspace = m->workspace; a.workspace_bytes = m->workspace_bytes; a.stream = m->stream;
  const TaWeights w = {wd, wd + C * C, wd + 2 * C * C, wd + 3 * C * C};
  return triatt_run<128, true>(&a, w);
}

extern "C" int pf_triatt_attend_workspace(void* workspace, size_t workspace_bytes, int B, int N, int n_valid,
                                          void* stream) {
  if (!workspace) return pf_fail(PF_E_INVALID, "pf_triatt_attend_workspace: null workspace");
  if (B <= 0 || N <= 0 || N % 64)
    return pf_fail(PF_E_INVALID, "pf_triatt_attend_workspace: need B > 0 and N a positive multiple of 64");
  if ((unsigned long long)B * N * N >= (1ull << 32) || !ta_shape_ok(N))
    return pf_fail(PF_E_INVALID, "pf_triatt_attend_workspace: need B * N * N < 2^32 and N <= 11584 (B=%d N=%d)",
                   B, N);
  if (n_valid < 0 || n_valid > N)
    return pf_fail(PF_E_INVALID, "pf_triatt_attend_workspace: n_valid %d outside [0, N=%d]", n_valid, N);
  const size_t need = ta_buffers_size(B, N);
  if (workspace_bytes < need)
    return pf_fail(PF_E_INVALID, "pf_triatt_attend_workspace: workspace too small (%zu < %zu bytes)",
                   workspace_bytes, need);
  return launch_attn<false>(ta_buffers(workspace, B, N), nullptr, B, N, n_valid ? n_valid : N, (hipStream_t)stream);
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
  if ((unsigned long long)B * N * N >= (1ull << 32) || !ta_shape_ok(N))
    return pf_fail(PF_E_INVALID, "pf_tri_attention: need B * N * N < 2^32 and N <= 11584 (B=%d N=%d)", B, N);
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
  ta_prep_qkv_kernel<<<(unsigned)(rows * (N / PREP_KB)), 256, 0, st>>>(q, k, v, scale * LOG2E, t.Q, t.K, t.Vt, N);
  PF_CHECK_LAUNCH("ta_prep_qkv_kernel");
  ta_prep_bias_kernel<<<1024, 256, 0, st>>>(bias, mask, t.bias32, t.mask16, (long)B * H * N * N, (long)B * N * N,
                                            N, n_valid);
  PF_CHECK_LAUNCH("ta_prep_bias_kernel");
  return launch_attn<true>(t, o, B, N, n_valid, st);
}
