// Fast mode (block fp8) for gfx950: MXFP8 e4m3 operands with one E8M0 scale per 32
// elements along every contraction axis, fp32 accumulation (v_mfma_scale_f32_32x32x64_f8f6f4).
//
// Replaces the --fast path of the ttnn TriangleMultiplication / Transition
// (tt_bio/tenstorrent.py:60-61, 178-181, 389-407, 431-503, 879-906), which stores these
// operands as Tenstorrent bfloat8_b; this build uses the OCP MX format instead (format and
// rounding in pf_common.h).  Quantization points:
//   triangle multiplication: LN_in(z) and p_in/g_in (K = 128 channels); the gated a/b
//     values along the contraction index k (the operand planes); LN_out(x) and p_out,
//     LN_in(z) and g_out (K = 128).  The contraction output x is stored as fp16 * 2^-8.
//   pair transition: LN(z) and fc1/fc2 (K = 128); silu(fc1)*fc2 and fc3 (K = 512).
// Everything else (LayerNorm statistics, gates, residual stream) is fp32.
//
//   mx8_quantize_kernel  rows x K fp32 -> e4m3 bytes + E8M0 scales (weights, tests)
//   tm8_proj_kernel      LN_in -> fp8 p_in|g_in -> a = p*sigmoid(g)*mask -> MXFP8 planes
//   tm8_contract_kernel  X[p][i][j] = sum_k A[p][i][k] B[p][j][k], MXFP8 operands
//   tm8_out_kernel       LN_out(X), LN_in(z) -> fp8 p_out / g_out -> gate -> residual
//   tr8_pair_kernel      LN -> fp8 fc1|fc2 -> silu*mul -> MXFP8 -> fp8 fc3 -> residual
#include "pf_common.h"
#include "pf_internal.h"

namespace {

constexpr int C = 128;
constexpr int WROW = 144;      // LDS pitch (bytes) of a 128-byte fp8 weight row: 9 x 16 B

// ---------------------------------------------------------------------------------
// Activation fragment of one 128-channel vector: lane (position m, half h) holds the
// channels 32j + 16h + t (j = 0..3 = channel block, t = 0..15).  As an MFMA operand
// for K step s (channels 64s .. 64s+63) the lane supplies bytes of blocks 2s and 2s+1
// and the scale of block 2s + h.
// ---------------------------------------------------------------------------------
struct X8 {
  i32x8 q[2];
  int sc[2];
};

PF_DEV void load_row128_x8order(const float* __restrict__ p, int h, float (&x)[4][16]) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(p + 32 * j + 16 * h + 4 * v);
      x[j][4 * v + 0] = a[0]; x[j][4 * v + 1] = a[1]; x[j][4 * v + 2] = a[2]; x[j][4 * v + 3] = a[3];
    }
}

// Quantize one 16-value slice of an MX block (the partner lane ^ 32 holds the other 16):
// returns the packed bytes and the block's scale byte.
PF_DEV i32x4 quantize16(const float (&y)[16], int& byte) {
  float a = amax16(y);
  a = xor32_max(a);
  byte = mx_scale_byte(a);
  return e4m3_pack16(y, mx_inv_scale(byte));
}

// LayerNorm (two-pass fp32, like ln128_to_frag) of a 128-vector in x8 order, quantized
// block by block (only one block of normalized values is live at a time).
PF_DEV void ln128_to_x8(const float (&x)[4][16], int h, const float* __restrict__ w,
                        const float* __restrict__ b, float eps, X8& out) {
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int t = 0; t < 16; ++t) s += x[j][t];
  const float mean = xor32_sum(s) * (1.f / 128.f);
  float v = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int t = 0; t < 16; ++t) { const float d = x[j][t] - mean; v += d * d; }
  const float rstd = rsqrtf(xor32_sum(v) * (1.f / 128.f) + eps);
  i32x4 q[4];
  int byte[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float y[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int c = 32 * j + 16 * h + t;
      y[t] = (x[j][t] - mean) * rstd * w[c] + b[c];
    }
    q[j] = quantize16(y, byte[j]);
  }
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    out.q[s2] = cat_i32x4(q[2 * s2], q[2 * s2 + 1]);
    out.sc[s2] = h ? byte[2 * s2 + 1] : byte[2 * s2];
  }
}

// The same LayerNorm with gamma and beta staged in LDS as [128] floats each, beta 512 bytes after
// gamma.  `lane_base` is the LDS byte address of gamma + 64 h (the lane half's first channel),
// held in one register so that every read is that register plus an immediate offset.
PF_DEV void ln128_to_x8_lds(const float (&x)[4][16], uint32_t lane_base, float eps, X8& out, int h) {
  typedef __attribute__((address_space(3))) const f32x4* lds_f4;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int t = 0; t < 16; ++t) s += x[j][t];
  const float mean = xor32_sum(s) * (1.f / 128.f);
  float v = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int t = 0; t < 16; ++t) { const float d = x[j][t] - mean; v += d * d; }
  const float rstd = rsqrtf(xor32_sum(v) * (1.f / 128.f) + eps);
  i32x4 q[4];
  int byte[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float y[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 w = *(lds_f4)(uintptr_t)(lane_base + 4 * (32 * j + 4 * g));
      const f32x4 b = *(lds_f4)(uintptr_t)(lane_base + 512 + 4 * (32 * j + 4 * g));
#pragma unroll
      for (int e = 0; e < 4; ++e) y[4 * g + e] = (x[j][4 * g + e] - mean) * rstd * w[e] + b[e];
    }
    q[j] = quantize16(y, byte[j]);
  }
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    out.q[s2] = cat_i32x4(q[2 * s2], q[2 * s2 + 1]);
    out.sc[s2] = h ? byte[2 * s2 + 1] : byte[2 * s2];
  }
}
PF_DEV uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)p;
}

// Weight fragment (MFMA operand) of row `row` of an fp8 [rows][128] matrix staged in LDS
// with pitch WROW, K step s, plus its scale byte (scales staged as [rows][4]).
PF_DEV i32x8 wfrag128(const uint8_t* lds, int row, int s, int h) {
  const uint8_t* p = lds + row * WROW + 64 * s + 16 * h;
  return cat_i32x4(*reinterpret_cast<const i32x4*>(p), *reinterpret_cast<const i32x4*>(p + 32));
}

// Copy an fp8 [rows][128] matrix (and its [rows][4] scales) from global to LDS.
PF_DEV void stage_w128(const uint8_t* __restrict__ q, const uint8_t* __restrict__ sc, int rows, uint8_t* lq,
                       uint8_t* ls, int tid, int nthreads) {
  for (int c = tid; c < rows * 8; c += nthreads)
    *reinterpret_cast<i32x4*>(lq + (c >> 3) * WROW + (c & 7) * 16) =
        *reinterpret_cast<const i32x4*>(q + (c >> 3) * 128 + (c & 7) * 16);
  for (int c = tid; c < rows; c += nthreads)
    *reinterpret_cast<int*>(ls + 4 * c) = *reinterpret_cast<const int*>(sc + 4 * c);
}

// ---------------------------------------------------------------------------------
// Quantize rows of K fp32 values in blocks of 32 along K.  One thread per block.
// perm = 1 stores each block in the order its values come out of a 32x32 MFMA
// accumulator pair (element 16h + 4j + e <- 4h + 8j + e), the column order of fc3.
// ---------------------------------------------------------------------------------
__global__ void mx8_quantize_kernel(const float* __restrict__ x, uint8_t* __restrict__ q,
                                    uint8_t* __restrict__ scales, long nblocks, int perm) {
  for (long blk = (long)blockIdx.x * blockDim.x + threadIdx.x; blk < nblocks; blk += (long)gridDim.x * blockDim.x) {
    const float* src = x + blk * 32;
    float v[32];
#pragma unroll
    for (int d = 0; d < 32; ++d) {
      const int s = perm ? 4 * (d >> 4) + 8 * ((d >> 2) & 3) + (d & 3) : d;
      v[d] = src[s];
    }
    float a = 0.f;
#pragma unroll
    for (int d = 0; d < 32; ++d) a = fmaxf(a, fabsf(v[d]));
    const int byte = mx_scale_byte(a);
    const float inv = mx_inv_scale(byte);
    int w[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) w[d] = e4m3_pack4(v[4 * d] * inv, v[4 * d + 1] * inv, v[4 * d + 2] * inv, v[4 * d + 3] * inv);
    i32x4* dst = reinterpret_cast<i32x4*>(q + blk * 32);
    dst[0] = i32x4{w[0], w[1], w[2], w[3]};
    dst[1] = i32x4{w[4], w[5], w[6], w[7]};
    scales[blk] = (uint8_t)byte;
  }
}

// ---------------------------------------------------------------------------------
// Triangle multiplication input projection.  One wave = 32 consecutive positions of
// one operand-plane row; p_in / g_in ([256][128] fp8 each) resident in LDS.  The
// projection is computed as D[position][channel], so a lane holds one channel for 16
// of the 32 positions and the partner lane the other 16: the MX block of the
// contraction (32 consecutive k = positions) is reduced with one exchange.  The LayerNorm's
// gamma / beta sit in LDS after the weights; the next tile's z rows (and mask entry) are
// loaded while a tile is computed; MASKED = false skips the mask.
//   A8/B8 planes [B][128][N][N] e4m3, scales SA/SB [B][128][N][N/32] E8M0.
// ---------------------------------------------------------------------------------
constexpr size_t TM8P_LDS = 2 * 256 * WROW + 2 * 256 * 4 + 2 * C * 4;   // + LayerNorm gamma, beta

template <bool MASKED>
__global__ __launch_bounds__(256, 2) void tm8_proj_kernel(
    const float* __restrict__ z, const float* __restrict__ mask, const float* __restrict__ lnw,
    const float* __restrict__ lnb, const uint8_t* __restrict__ wp_q, const uint8_t* __restrict__ wp_s,
    const uint8_t* __restrict__ wg_q, const uint8_t* __restrict__ wg_s, uint8_t* __restrict__ A8,
    uint8_t* __restrict__ B8, uint8_t* __restrict__ SA, uint8_t* __restrict__ SB, int B, int N, int incoming,
    float eps) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];
  uint8_t* lp = lds8;
  uint8_t* lg = lp + 256 * WROW;
  uint8_t* lps = lg + 256 * WROW;
  uint8_t* lgs = lps + 256 * 4;
  float* lnp = reinterpret_cast<float*>(lgs + 256 * 4);   // gamma [128], beta [128]
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, m = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  stage_w128(wp_q, wp_s, 256, lp, lps, tid, 256);
  stage_w128(wg_q, wg_s, 256, lg, lgs, tid, 256);
  if (tid < C) {
    lnp[tid] = lnw[tid];
    lnp[C + tid] = lnb[tid];
  }
  __syncthreads();

  uint32_t ln_a = lds_addr(lnp) + 64 * h;   // gamma of this lane half's first channel
  asm volatile("" : "+v"(ln_a));
  const uint32_t ntiles = (uint32_t)B * N * N / 32;
  const uint32_t stride = gridDim.x * 4;
  const int NB = N / 32;
  auto zpair = [&](uint32_t tile) -> long {
    const PosTile pt = pos_tile(tile, N);
    const int zi = incoming ? pt.c0 + m : pt.r;
    const int zj = incoming ? pt.r : pt.c0 + m;
    return ((long)pt.b * N + zi) * N + zj;
  };
  // the next tile's z row (and mask entry) are loaded while this tile is computed
  float xn[4][16];
  float mn = 1.f;
  uint32_t tile = blockIdx.x * 4 + wid;
  if (tile < ntiles) {
    const long pair = zpair(tile);
    load_row128_x8order(z + pair * C, h, xn);
    if (MASKED) mn = mask[pair];
  }
  for (; tile < ntiles; tile += stride) {
    // the LayerNorm parameters are re-read from LDS each tile instead of pinning 128 VGPRs
    asm volatile("" ::: "memory");
    const PosTile pt = pos_tile(tile, N);
    const int b = pt.b, orow = pt.r, ocol0 = pt.c0;
    X8 xq;
    float mr[16];
    {
      float x[4][16];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int t = 0; t < 16; ++t) x[j][t] = xn[j][t];
      const float maskv = mn;
      if (tile + stride < ntiles) {
        const long pair2 = zpair(tile + stride);
        load_row128_x8order(z + pair2 * C, h, xn);
        if (MASKED) mn = mask[pair2];
      }
      ln128_to_x8_lds(x, ln_a, eps, xq, h);
      if (MASKED) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mr[r] = __shfl(maskv, acc_row(r, h));
      }
    }

    // unrolled, so that the next tile's wait for its prefetched rows can count the stores issued
    // after them; the empty asm keeps each block's LDS reads in its own block
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
      asm volatile("" ::: "memory");
      const int row = 32 * cb + m;   // weight row = output unit of this lane's column
      f32x16 P = zero16(), G = zero16();
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        P = mfma8(xq.q[s], wfrag128(lp, row, s, h), P, xq.sc[s], lps[4 * row + 2 * s + h]);
        G = mfma8(xq.q[s], wfrag128(lg, row, s, h), G, xq.sc[s], lgs[4 * row + 2 * s + h]);
      }
      float v[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        v[r] = P[r] * sigmoidf_fast(G[r]);
        if (MASKED) v[r] *= mr[r];
      }
      int byte;
      const i32x4 q = quantize16(v, byte);
      const int ch = 32 * (cb & 3) + m;
      uint8_t* plane = (cb < 4 ? A8 : B8) + (((long)b * C + ch) * N + orow) * N + ocol0;
      // dword g of lane half h holds positions 8g + 4h .. +3; one v_permlane32_swap per
      // dword pair gives half 0 positions 0..15 and half 1 positions 16..31, so the
      // 32-byte plane-row segment leaves as two 16-byte stores instead of eight 4-byte ones
      i32x4 o;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        // r[1] on half 0 = half 1's q[k]; r[0] on half 1 = half 0's q[2+k]
        const auto r = __builtin_amdgcn_permlane32_swap(q[k], q[2 + k], false, false);
        o[2 * k] = h ? (int)r[0] : q[k];
        o[2 * k + 1] = h ? q[2 + k] : (int)r[1];
      }
      *reinterpret_cast<i32x4*>(plane + 16 * h) = o;
      if (h == 0) (cb < 4 ? SA : SB)[(((long)b * C + ch) * N + orow) * NB + ocol0 / 32] = (uint8_t)byte;
    }
  }
}

// ---------------------------------------------------------------------------------
// Contraction X[p][i][j] = sum_k A[p][i][k] * B[p][j][k] on MXFP8 planes.
// 256x256 output tile per workgroup of 8 waves (two per SIMD), each 128 (i) x 64 (j), as
// the 16-bit kernel; slabs of 128 k (128 bytes per row) move global -> LDS by DMA through a
// 2-deep ring with the same XOR row swizzle.  The slab's scale dwords (the 4 blocks of each
// row) travel with it by DMA (one 4-byte-per-lane instruction per wave: waves 0-3 the A rows,
// 4-7 the B rows), into [row][4 bytes] after the two operand slabs of the stage; loaded into
// registers with ordinary global loads instead, they held every slab's wait back (+30 % at
// N = 1024).
// ---------------------------------------------------------------------------------
constexpr int BT = 256, SK = 128, TM8C_WAVES = 8;
constexpr int SLAB8 = BT * SK;                        // bytes per operand slab
constexpr int SCL8 = 2 * BT * 4;                      // the slab's scale dwords, A rows then B rows
constexpr int STAGE8 = 2 * SLAB8 + SCL8;              // bytes per ring stage
constexpr size_t TM8C_LDS = (size_t)2 * STAGE8;
PF_DEV int slab_swz8(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }

template <typename OutT>
__global__ __launch_bounds__(64 * TM8C_WAVES, 1) void tm8_contract_kernel(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ Bop, const uint8_t* __restrict__ SA,
    const uint8_t* __restrict__ SB, OutT* __restrict__ X, int N, int tpd, int total, float out_scale) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem8[];
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, m = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid >> 2, wn = wid & 3;
  const int w = xcd_remap(blockIdx.x, total);
  const int tiles = tpd * tpd;
  const long plane = w / tiles;
  const int t = w - (int)plane * tiles;
  const int i0 = (t / tpd) * BT, j0 = (t % tpd) * BT;
  const long NN = (long)N * N;
  const int NB = N / 32;

  // DMA: instruction q (0..3) of this wave covers slab rows (4*wid + q)*8 + (lane >> 3)
  int offA[4], offB[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (4 * wid + q) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ slab_swz8(r);
    offA[q] = min(i0 + r, N - 1) * N + 16 * c;
    offB[q] = min(j0 + r, N - 1) * N + 16 * c;
  }
  const uint8_t* Ap = A + plane * NN;
  const uint8_t* Bp = Bop + plane * NN;
  // scale DMA: wave w < 4 moves A rows 64 w + lane, wave w >= 4 B rows 64 (w - 4) + lane (a
  // 32-bit offset from SA / SB: fewer registers than a pointer)
  const uint8_t* Sp = wid < 4 ? SA : SB;
  const int srow = (wid & 3) * 64 + lane;
  const int sOff = (int)((plane * N + min((wid < 4 ? i0 : j0) + srow, N - 1)) * NB);
  auto issue = [&](int kt) {
    uint8_t* sa = smem8 + (kt & 1) * STAGE8;
    uint8_t* sb = sa + SLAB8;
    const int ko = kt * SK;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      __builtin_amdgcn_global_load_lds(Ap + offA[q] + ko, sa + (4 * wid + q) * 1024, 16, 0, 0);
      __builtin_amdgcn_global_load_lds(Bp + offB[q] + ko, sb + (4 * wid + q) * 1024, 16, 0, 0);
    }
    __builtin_amdgcn_global_load_lds(Sp + sOff + 4 * kt, sa + 2 * SLAB8 + 256 * wid, 4, 0, 0);
  };
  // this lane's scale dwords of a stage: A rows wm*128 + 32x + m, B rows wn*64 + 32y + m
  int scA[4], scB[2];
  auto read_scales = [&](int kt) {
    const uint8_t* ss = smem8 + (kt & 1) * STAGE8 + 2 * SLAB8;
#pragma unroll
    for (int x = 0; x < 4; ++x) scA[x] = *reinterpret_cast<const int*>(ss + 4 * (wm * 128 + 32 * x + m));
#pragma unroll
    for (int y = 0; y < 2; ++y) scB[y] = *reinterpret_cast<const int*>(ss + 4 * BT + 4 * (wn * 64 + 32 * y + m));
  };
  const int swz = slab_swz8(m);
  const int rdA = (wm * 128 + m) * SK, rdB = (wn * 64 + m) * SK;
  auto read_frags = [&](int kt, int s, i32x8 (&fa)[4], i32x8 (&fb)[2]) {
    const uint8_t* sa = smem8 + (kt & 1) * STAGE8;
    const uint8_t* sb = sa + SLAB8;
    const int c0 = 16 * ((4 * s + h) ^ swz), c1 = 16 * ((4 * s + 2 + h) ^ swz);
#pragma unroll
    for (int x = 0; x < 4; ++x)
      fa[x] = cat_i32x4(*reinterpret_cast<const i32x4*>(sa + rdA + 32 * x * SK + c0),
                        *reinterpret_cast<const i32x4*>(sa + rdA + 32 * x * SK + c1));
#pragma unroll
    for (int y = 0; y < 2; ++y)
      fb[y] = cat_i32x4(*reinterpret_cast<const i32x4*>(sb + rdB + 32 * y * SK + c0),
                        *reinterpret_cast<const i32x4*>(sb + rdB + 32 * y * SK + c1));
  };
  f32x16 acc[2][4];
#pragma unroll
  for (int y = 0; y < 2; ++y)
#pragma unroll
    for (int x = 0; x < 4; ++x) acc[y][x] = zero16();

  const int nk = N / SK;
  issue(0);
  for (int kt = 0; kt < nk; ++kt) {
    // slab kt and its scales landed; the barrier also frees slab kt-1's buffer
    __builtin_amdgcn_s_waitcnt(vmcnt_le(0));
    __builtin_amdgcn_s_barrier();
    if (kt + 1 < nk) issue(kt + 1);
    __builtin_amdgcn_sched_barrier(0);
    read_scales(kt);
    // k-step 0's fragments, then step 1's reads interleaved with step 0's MFMAs (two reads
    // after each of the first six), then step 1's MFMAs
    i32x8 f0a[4], f0b[2], f1a[4], f1b[2];
    read_frags(kt, 0, f0a, f0b);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(kt, 1, f1a, f1b);
    {
      const int sh = 8 * h;
#pragma unroll
      for (int y = 0; y < 2; ++y)
#pragma unroll
        for (int x = 0; x < 4; ++x)
          acc[y][x] = mfma8(f0b[y], f0a[x], acc[y][x], (scB[y] >> sh) & 0xFF, (scA[x] >> sh) & 0xFF);
    }
#pragma unroll
    for (int q = 0; q < 6; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __builtin_amdgcn_sched_barrier(0);
    {
      const int sh = 8 * (2 + h);
#pragma unroll
      for (int y = 0; y < 2; ++y)
#pragma unroll
        for (int x = 0; x < 4; ++x)
          acc[y][x] = mfma8(f1b[y], f1a[x], acc[y][x], (scB[y] >> sh) & 0xFF, (scA[x] >> sh) & 0xFF);
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  OutT* Xp = X + plane * NN;
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int ib = i0 + wm * 128 + 32 * x;
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int jb = j0 + wn * 64 + 32 * y;
      if (ib >= N || jb >= N) continue;
      if constexpr (sizeof(OutT) == 4) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          f32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[y][x][4 * g + e] * out_scale;
          *reinterpret_cast<f32x4*>(Xp + (long)(ib + m) * N + jb + 8 * g + 4 * h) = v;
        }
      } else {
        store_runs16((op_t*)(Xp + (long)(ib + m) * N + jb), acc[y][x], out_scale, h);   // 16-byte runs
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Triangle multiplication output: z[i,j,:] (+)= p_out(q(LN_out(X))) * sigmoid(g_out(q(LN_in(z)))).
// Persistent; a workgroup takes 128 consecutive pairs (i, j0..j0+127) per step: the X slice
// X[b][0..127][i][j0..j0+127] (32 KB, 256-byte rows) is loaded a step ahead into registers
// (16-byte loads), written to LDS and read back channel by channel; wave w owns pairs
// j0 + 32w .. j0 + 32w + 31.  p_out/g_out ([128][128] fp8, rows half-major) and both
// LayerNorms' parameters stay in LDS.  The projections run as D[channel][pair], so a lane
// half holds 16 consecutive output channels of its pair: the z row it loaded for LN_in is the
// residual and every store is a 64-byte run.
// ---------------------------------------------------------------------------------
constexpr int XP = 136;        // LDS pitch (halves) of one channel row of the X slice
constexpr size_t TM8O_LDS = 2 * 128 * WROW + 2 * 128 * 4 + (size_t)C * XP * 2 + 4 * C * 4;

// Stage an fp8 [128][128] matrix (and its [128][4] scales) from global to LDS with the rows
// of each 32-row block permuted: LDS row 32 o + 8 q + 4 h + e holds row 32 o + 16 h + 4 q + e.
// A 32x32 MFMA with these rows as its A operand then leaves, in lane half h, register r, the
// output channel 32 o + 16 h + r: a lane half owns 16 consecutive channels per block.
PF_DEV int half_major_row(int R) { return (R & ~31) + 16 * ((R >> 2) & 1) + 4 * ((R >> 3) & 3) + (R & 3); }
PF_DEV void stage_w128_half_major(const uint8_t* __restrict__ q, const uint8_t* __restrict__ sc, uint8_t* lq,
                                  uint8_t* ls, int tid, int nthreads) {
  for (int c = tid; c < 128 * 8; c += nthreads)
    *reinterpret_cast<i32x4*>(lq + (c >> 3) * WROW + (c & 7) * 16) =
        *reinterpret_cast<const i32x4*>(q + half_major_row(c >> 3) * 128 + (c & 7) * 16);
  for (int c = tid; c < 128; c += nthreads)
    *reinterpret_cast<int*>(ls + 4 * c) = *reinterpret_cast<const int*>(sc + 4 * half_major_row(c));
}

// RESID: 0 = no residual (out = update), 1 = out is z_in (the LN_in row is the residual),
// 2 = out += update (out distinct from z_in)
template <typename XT, int RESID>
__global__ __launch_bounds__(256, 2) void tm8_out_kernel(
    const XT* __restrict__ X, float x_scale, const float* z_in, float* out, const float* __restrict__ lni_w,
    const float* __restrict__ lni_b, const float* __restrict__ lno_w, const float* __restrict__ lno_b,
    const uint8_t* __restrict__ wp_q, const uint8_t* __restrict__ wp_s, const uint8_t* __restrict__ wg_q,
    const uint8_t* __restrict__ wg_s, int B, int N, float eps) {
  static_assert(sizeof(XT) == 2, "X slice staging assumes 16-bit X");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];
  uint8_t* lp = lds8;
  uint8_t* lg = lp + 128 * WROW;
  uint8_t* lps = lg + 128 * WROW;
  uint8_t* lgs = lps + 128 * 4;
  XT* lx = reinterpret_cast<XT*>(lgs + 128 * 4);
  float* lnp = reinterpret_cast<float*>(lx + C * XP);   // LN_out gamma, beta, LN_in gamma, beta
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, h = lane >> 5, m = lane & 31;
  stage_w128_half_major(wp_q, wp_s, lp, lps, tid, 256);
  stage_w128_half_major(wg_q, wg_s, lg, lgs, tid, 256);
  if (tid < C) {
    lnp[tid] = lno_w[tid];
    lnp[C + tid] = lno_b[tid];
    lnp[2 * C + tid] = lni_w[tid];
    lnp[3 * C + tid] = lni_b[tid];
  }
  uint32_t ln_o = lds_addr(lnp) + 64 * h, ln_i = ln_o + 1024;   // LN_out / LN_in gamma of this half
  asm volatile("" : "+v"(ln_o), "+v"(ln_i));

  const long NN = (long)N * N;
  const long nsteps = (long)B * NN / 128;
  // X slice of a step: thread tid moves chunks tid + 256 q (channel c >> 4, 8 pairs at (c & 15) * 8)
  auto x_src = [&](long step) -> const XT* {
    const long pair0 = step * 128;
    const long b = pair0 / NN;
    return X + b * C * NN + (pair0 - b * NN);
  };
  opx8 xr[8];   // the next step's X chunks, in flight during this step
  long step = blockIdx.x;
  if (step < nsteps) {
    const XT* src = x_src(step);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int c = tid + 256 * q;
      xr[q] = *reinterpret_cast<const opx8*>(src + (long)(c >> 4) * NN + (c & 15) * 8);
    }
  }
  for (; step < nsteps; step += gridDim.x) {
    asm volatile("" ::: "memory");               // LayerNorm parameters are re-read, not pinned
    const long pos0 = step * 128 + 32 * wid;     // this wave's 32 pairs
    float zr[4][16];                             // LN_in input and (resid 1) the residual
    load_row128_x8order(z_in + (pos0 + m) * C, h, zr);
    __syncthreads();                             // previous step's readers are done
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int c = tid + 256 * q;
      *reinterpret_cast<opx8*>(lx + (c >> 4) * XP + (c & 15) * 8) = xr[q];
    }
    if (step + gridDim.x < nsteps) {             // issued after the z row: its wait does not cover these
      const XT* src = x_src(step + gridDim.x);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int c = tid + 256 * q;
        xr[q] = *reinterpret_cast<const opx8*>(src + (long)(c >> 4) * NN + (c & 15) * 8);
      }
    }
    __syncthreads();
    X8 xo, xi;
    {
      float x[4][16];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int tt = 0; tt < 16; ++tt) x[j][tt] = (float)lx[(32 * j + 16 * h + tt) * XP + 32 * wid + m] * x_scale;
      ln128_to_x8_lds(x, ln_o, eps, xo, h);
    }
    ln128_to_x8_lds(zr, ln_i, eps, xi, h);
    // D[channel][pair] with half-major weight rows: lane (pair m, half h) holds channels
    // 32 ob + 16 h + r, 64 contiguous bytes of its output row, the same channels as zr[ob]
    float* orow = out + (pos0 + m) * C + 16 * h;
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) {
      asm volatile("" ::: "memory");   // keeps each block's LDS fragment reads in its block
      const int row = 32 * ob + m;
      f32x16 P = zero16(), G = zero16();
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        P = mfma8(wfrag128(lp, row, s, h), xo.q[s], P, lps[4 * row + 2 * s + h], xo.sc[s]);
        G = mfma8(wfrag128(lg, row, s, h), xi.q[s], G, lgs[4 * row + 2 * s + h], xi.sc[s]);
      }
      f32x4 res[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (RESID == 2) res[q] = *reinterpret_cast<const f32x4*>(orow + 32 * ob + 4 * q);
        else if (RESID == 1) res[q] = f32x4{zr[ob][4 * q], zr[ob][4 * q + 1], zr[ob][4 * q + 2], zr[ob][4 * q + 3]};
        else res[q] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = P[4 * q + e] * sigmoidf_fast(G[4 * q + e]) + res[q][e];
        *reinterpret_cast<f32x4*>(orow + 32 * ob + 4 * q) = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Pair transition, MXFP8.  A workgroup is 4 waves x 32 pairs; three workgroups share a CU
// (<= 168 VGPRs).  Per block of 64 hidden units the fp8 fc1 / fc2 rows ([64][128] bytes),
// the fc3 column slice ([128][64] bytes) and their scale bytes move global -> LDS by DMA
// (global_load_lds, no VGPR staging) into a 2-stage ring, one barrier per block.  Rows
// are unpadded with XOR-swizzled 16-byte chunks (fc1 / fc2: chunk c of row R at slot
// c ^ swz8(R); fc3: c ^ swz4(R)) so fragment reads are conflict-free.  fc1 / fc2 run as
// D[hidden][pair]; silu(a)*b is quantized per 32 hidden units (one lane-half exchange)
// and is directly fc3's B operand (fc3.weight is stored in accumulator order, perm = 1);
// fc3 runs as D[channel][pair], so a lane owns one pair and the residual update is
// 16-byte loads and stores in the output-aligned layout.
// ---------------------------------------------------------------------------------
constexpr int TR8_W1 = 0, TR8_W2 = 8192, TR8_W3 = 16384, TR8_S1 = 24576, TR8_S2 = 24832, TR8_S3 = 25088;
constexpr int TR8_STAGE = 25600;   // bytes of one ring stage
PF_DEV int tr8_swz8(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }
PF_DEV int tr8_swz4(int r) { return (r >> 2) & 3; }

template <bool ZBIAS>
__global__ __launch_bounds__(256, 3) void tr8_pair_kernel(
    const float* x_in, float* out, const float* __restrict__ lnw, const float* __restrict__ lnb,
    const uint8_t* __restrict__ w1q, const uint8_t* __restrict__ w1s, const uint8_t* __restrict__ w2q,
    const uint8_t* __restrict__ w2s, const uint8_t* __restrict__ w3q, const uint8_t* __restrict__ w3s,
    long rows, int hidden, int accumulate, float eps, ZBiasArgs zb) {
  __shared__ __attribute__((aligned(16))) uint8_t tl[2 * TR8_STAGE];
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, m = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const long pos0 = ((long)blockIdx.x * 4 + wid) * 32;
  const int nblk = hidden / 32;   // MX blocks along the hidden axis (a multiple of 4)

  X8 xq;
  {
    float x[4][16];
    load_row128_x8order(x_in + min(pos0 + m, rows - 1) * C, h, x);
    ln128_to_x8(x, h, lnw, lnb, eps, xq);
  }
  f32x16 acc[4];
#pragma unroll
  for (int ob = 0; ob < 4; ++ob) acc[ob] = zero16();

  // DMA: wave w moves 1 KB pieces 2w and 2w+1 of each 8 KB matrix block, plus one piece
  // of scales (w = 0: fc1, 1: fc2, 2 / 3: fc3 rows 0-63 / 64-127, one dword per row)
  uint32_t o12[2], o3[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int R = 8 * (2 * wid + i) + (lane >> 3);
    o12[i] = (uint32_t)(R * C + 16 * ((lane & 7) ^ tr8_swz8(R)));
    const int R3 = 16 * (2 * wid + i) + (lane >> 2);
    o3[i] = (uint32_t)(R3 * hidden + 16 * ((lane & 3) ^ tr8_swz4(R3)));
  }
  auto issue = [&](int hp, int buf) PF_INLINE {
    uint8_t* st = tl + buf * TR8_STAGE;
    const uint8_t* b1 = w1q + (long)64 * hp * C;
    const uint8_t* b2 = w2q + (long)64 * hp * C;
    const uint8_t* b3 = w3q + 64 * hp;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int piece = 1024 * (2 * wid + i);
      __builtin_amdgcn_global_load_lds(b1 + o12[i], st + TR8_W1 + piece, 16, 0, 0);
      __builtin_amdgcn_global_load_lds(b2 + o12[i], st + TR8_W2 + piece, 16, 0, 0);
      __builtin_amdgcn_global_load_lds(b3 + o3[i], st + TR8_W3 + piece, 16, 0, 0);
    }
    if (wid == 0) __builtin_amdgcn_global_load_lds(w1s + 256 * hp + 4 * lane, st + TR8_S1, 4, 0, 0);
    else if (wid == 1) __builtin_amdgcn_global_load_lds(w2s + 256 * hp + 4 * lane, st + TR8_S2, 4, 0, 0);
    else
      __builtin_amdgcn_global_load_lds(w3s + (long)(64 * (wid - 2) + lane) * nblk + 4 * (hp >> 1),
                                       st + TR8_S3 + 256 * (wid - 2), 4, 0, 0);
  };
  const int sw8 = tr8_swz8(m), sw4 = tr8_swz4(m);   // rows 32x + m share the low 4 bits of m

  const int nhp = hidden / 64;
  issue(0, 0);
  for (int hp = 0; hp < nhp; ++hp) {
    __builtin_amdgcn_s_waitcnt(vmcnt_le(0));   // block hp landed ...
    __builtin_amdgcn_s_barrier();              // ... for every wave; the other stage is free
    asm volatile("" ::: "memory");
    if (hp + 1 < nhp) issue(hp + 1, (hp + 1) & 1);
    const uint8_t* st = tl + (hp & 1) * TR8_STAGE;
    i32x4 hq[2];
    int hbyte[2];
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      const int row = 32 * bb + m;   // hidden unit 64 hp + row
      f32x16 a1 = zero16(), a2 = zero16();
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int c0 = ((4 * s + h) ^ sw8) * 16, c1 = ((4 * s + h + 2) ^ sw8) * 16;
        const uint8_t* r1 = st + TR8_W1 + row * C;
        const uint8_t* r2 = st + TR8_W2 + row * C;
        const i32x8 f1 = cat_i32x4(*reinterpret_cast<const i32x4*>(r1 + c0), *reinterpret_cast<const i32x4*>(r1 + c1));
        const i32x8 f2 = cat_i32x4(*reinterpret_cast<const i32x4*>(r2 + c0), *reinterpret_cast<const i32x4*>(r2 + c1));
        a1 = mfma8(f1, xq.q[s], a1, st[TR8_S1 + 4 * row + 2 * s + h], xq.sc[s]);
        a2 = mfma8(f2, xq.q[s], a2, st[TR8_S2 + 4 * row + 2 * s + h], xq.sc[s]);
      }
      float v[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) v[r] = siluf(a1[r]) * a2[r];
      hq[bb] = quantize16(v, hbyte[bb]);
      __builtin_amdgcn_sched_barrier(0);   // keep the next half's fragment reads after this one (registers)
    }
    const i32x8 hop = cat_i32x4(hq[0], hq[1]);
    const int hsc = h ? hbyte[1] : hbyte[0];
    const int sb = 2 * (hp & 1) + h;   // scale byte of K block h within the fc3 row dword
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) {
      const int orow = 32 * ob + m;
      const uint8_t* p = st + TR8_W3 + orow * 64;
      const i32x8 wf = cat_i32x4(*reinterpret_cast<const i32x4*>(p + 16 * (h ^ sw4)),
                                 *reinterpret_cast<const i32x4*>(p + 16 * ((h + 2) ^ sw4)));
      acc[ob] = mfma8(wf, hop, acc[ob], st[TR8_S3 + 4 * orow + sb], hsc);   // rows = channel, cols = pair
    }
  }
  pair_update_epilogue<ZBIAS>(acc, out, rows, pos0, m, h, accumulate, zb);
}

// Workspace layout of the fp8 triangle multiplication.
struct Tm8Buffers {
  uint8_t *A8, *B8, *SA, *SB;
  op_t* X;
};
size_t tm8_buffers_size(int B, int N) {
  const size_t planes = (size_t)B * C * N * N;
  return 2 * planes + 2 * (planes / 32) + planes * sizeof(op_t);
}
Tm8Buffers tm8_buffers(void* ws, int B, int N) {
  const size_t planes = (size_t)B * C * N * N;
  Tm8Buffers t;
  t.A8 = (uint8_t*)ws;
  t.B8 = t.A8 + planes;
  t.SA = t.B8 + planes;
  t.SB = t.SA + planes / 32;
  t.X = (op_t*)(t.SB + planes / 32);
  return t;
}

// grid of a wave-tile loop: enough workgroups to fill the chip several times over
int tile_grid(long ntiles) { const long g = (ntiles + 3) / 4; return (int)(g < 2048 ? g : 2048); }

}  // namespace

// ---------------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------------
extern "C" int pf_quantize_mx8(const float* x, long rows, int K, int perm, void* q, void* scales, void* stream) {
  if (!x || !q || !scales) return pf_fail(PF_E_INVALID, "pf_quantize_mx8: null pointer");
  if (rows <= 0 || K <= 0 || K % 32) return pf_fail(PF_E_INVALID, "pf_quantize_mx8: need rows > 0 and K a multiple of 32");
  if (perm != 0 && perm != 1) return pf_fail(PF_E_INVALID, "pf_quantize_mx8: perm must be 0 or 1");
  const long nblocks = rows * (K / 32);
  const long g = (nblocks + 255) / 256;
  const int grid = (int)(g < 4096 ? g : 4096);
  mx8_quantize_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(x, (uint8_t*)q, (uint8_t*)scales, nblocks, perm);
  PF_CHECK_LAUNCH("mx8_quantize_kernel");
  return PF_OK;
}

extern "C" size_t pf_trimul_mx8_workspace_size(int B, int N, int C_) {
  if (B <= 0 || N <= 0 || C_ != C) return 0;
  return tm8_buffers_size(B, N);
}

extern "C" int pf_trimul_mx8_fwd(const pf_trimul_mx8_args* a) {
  if (!a) return pf_fail(PF_E_INVALID, "pf_trimul_mx8_fwd: null args");
  if (a->C != C || a->hidden != C)
    return pf_fail(PF_E_INVALID, "pf_trimul_mx8_fwd: only c_z = hidden = 128 is supported (got %d, %d)", a->C, a->hidden);
  if (a->B <= 0 || a->N <= 0 || a->N % 128)
    return pf_fail(PF_E_INVALID, "pf_trimul_mx8_fwd: need B > 0 and N a positive multiple of 128 (B=%d N=%d)",
                   a->B, a->N);
  if ((unsigned long long)a->B * a->N * a->N >= (1ull << 32))
    return pf_fail(PF_E_INVALID, "pf_trimul_mx8_fwd: B * N * N must be below 2^32 (B=%d N=%d)", a->B, a->N);
  if (a->direction != 0 && a->direction != 1)
    return pf_fail(PF_E_INVALID, "pf_trimul_mx8_fwd: direction must be 0 (outgoing) or 1 (incoming)");
  if (!a->z_in || !a->out || !a->norm_in_w || !a->norm_in_b || !a->p_in_q || !a->p_in_s || !a->g_in_q ||
      !a->g_in_s || !a->norm_out_w || !a->norm_out_b || !a->p_out_q || !a->p_out_s || !a->g_out_q ||
      !a->g_out_s || !a->workspace)
    return pf_fail(PF_E_INVALID, "pf_trimul_mx8_fwd: null pointer argument");
  if ((long)a->B * C * a->N * (a->N / 32) >= (1l << 31))   // scale bytes are addressed with 32-bit offsets
    return pf_fail(PF_E_INVALID, "pf_trimul_mx8_fwd: B * C * N * N / 32 must stay below 2^31 (B=%d N=%d)", a->B, a->N);
  const size_t need = tm8_buffers_size(a->B, a->N);
  if (a->workspace_bytes < need)
    return pf_fail(PF_E_INVALID, "pf_trimul_mx8_fwd: workspace too small (%zu < %zu bytes)", a->workspace_bytes, need);
  {
    int rc = pf_reserve_lds((const void*)tm8_proj_kernel<true>, TM8P_LDS, "tm8_proj_kernel");
    if (rc == PF_OK) rc = pf_reserve_lds((const void*)tm8_proj_kernel<false>, TM8P_LDS, "tm8_proj_kernel");
    if (rc == PF_OK) rc = pf_reserve_lds((const void*)tm8_contract_kernel<op_t>, TM8C_LDS, "tm8_contract_kernel");
    if (rc == PF_OK) rc = pf_reserve_lds((const void*)tm8_out_kernel<op_t, 0>, TM8O_LDS, "tm8_out_kernel");
    if (rc == PF_OK) rc = pf_reserve_lds((const void*)tm8_out_kernel<op_t, 1>, TM8O_LDS, "tm8_out_kernel");
    if (rc == PF_OK) rc = pf_reserve_lds((const void*)tm8_out_kernel<op_t, 2>, TM8O_LDS, "tm8_out_kernel");
    if (rc != PF_OK) return rc;
  }
  hipStream_t st = (hipStream_t)a->stream;
  const int B = a->B, N = a->N;
  Tm8Buffers t = tm8_buffers(a->workspace, B, N);
  const long ntiles = (long)B * N * N / 32;
  const int cus = device_cus();
  if (cus <= 0) return pf_fail(PF_E_LAUNCH, "pf_trimul_mx8_fwd: cannot query the device");
  // up to 2048 workgroups (several rounds per CU): a persistent grid of two per CU projects
  // as fast but leaves the planes in an order the contraction reads 6 % slower
  const int grid = tile_grid(ntiles);
  // the A plane (channels 0..127 of the projection) holds a, the B plane b; the
  // 2C-row p_in / g_in matrices are [a rows ; b rows]
  (a->pair_mask ? tm8_proj_kernel<true> : tm8_proj_kernel<false>)<<<grid, 256, TM8P_LDS, st>>>(
      a->z_in, a->pair_mask, a->norm_in_w, a->norm_in_b, (const uint8_t*)a->p_in_q, (const uint8_t*)a->p_in_s,
      (const uint8_t*)a->g_in_q, (const uint8_t*)a->g_in_s, t.A8, t.B8, t.SA, t.SB, B, N, a->direction, a->eps);
  PF_CHECK_LAUNCH("tm8_proj_kernel");
  const int tpd = (N + BT - 1) / BT;
  const int total = B * C * tpd * tpd;
  pf_kernel_mark(PF_TIMED_CONTRACT8, st, 0);
  tm8_contract_kernel<op_t><<<total, 64 * TM8C_WAVES, TM8C_LDS, st>>>(t.A8, t.B8, t.SA, t.SB, t.X, N, tpd, total, X_STORE_SCALE);
  pf_kernel_mark(PF_TIMED_CONTRACT8, st, 1);
  PF_CHECK_LAUNCH("tm8_contract_kernel");
  const long nsteps = (long)B * N * N / 128;
  // persistent: two 4-wave workgroups per CU, each staging the weights once
  const int resid = !a->accumulate ? 0 : (a->out == a->z_in ? 1 : 2);
  auto out_kern = resid == 0 ? tm8_out_kernel<op_t, 0> : resid == 1 ? tm8_out_kernel<op_t, 1> : tm8_out_kernel<op_t, 2>;
  out_kern<<<(int)min((long)2 * cus, nsteps), 256, TM8O_LDS, st>>>(
      t.X, X_LOAD_SCALE, a->z_in, a->out, a->norm_in_w, a->norm_in_b, a->norm_out_w, a->norm_out_b,
      (const uint8_t*)a->p_out_q, (const uint8_t*)a->p_out_s, (const uint8_t*)a->g_out_q, (const uint8_t*)a->g_out_s,
      B, N, a->eps);
  PF_CHECK_LAUNCH("tm8_out_kernel");
  return PF_OK;
}

extern "C" int pf_trimul_mx8_contract(const void* A8, const void* B8, const void* SA, const void* SB, float* X,
                                      int planes, int N, void* stream) {
  if (!A8 || !B8 || !SA || !SB || !X) return pf_fail(PF_E_INVALID, "pf_trimul_mx8_contract: null pointer");
  if (planes <= 0 || N <= 0 || N % 128)
    return pf_fail(PF_E_INVALID, "pf_trimul_mx8_contract: need planes > 0 and N a multiple of 128");
  if ((long)planes * N * (N / 32) >= (1l << 31))   // scale bytes are addressed with 32-bit offsets
    return pf_fail(PF_E_INVALID, "pf_trimul_mx8_contract: planes * N * N / 32 must stay below 2^31 (planes=%d N=%d)",
                   planes, N);
  if (const int rc = pf_reserve_lds((const void*)tm8_contract_kernel<float>, TM8C_LDS, "tm8_contract_kernel"))
    return rc;
  const int tpd = (N + BT - 1) / BT;
  const int total = planes * tpd * tpd;
  pf_kernel_mark(PF_TIMED_CONTRACT8, (hipStream_t)stream, 0);
  tm8_contract_kernel<float><<<total, 64 * TM8C_WAVES, TM8C_LDS, (hipStream_t)stream>>>(
      (const uint8_t*)A8, (const uint8_t*)B8, (const uint8_t*)SA, (const uint8_t*)SB, X, N, tpd, total, 1.f);
  pf_kernel_mark(PF_TIMED_CONTRACT8, (hipStream_t)stream, 1);
  PF_CHECK_LAUNCH("tm8_contract_kernel");
  return PF_OK;
}

extern "C" int pf_transition_mx8_fwd(const pf_transition_mx8_args* a) {
  if (!a) return pf_fail(PF_E_INVALID, "pf_transition_mx8_fwd: null args");
  if (a->C != C || a->hidden <= 0 || a->hidden % 128)
    return pf_fail(PF_E_INVALID, "pf_transition_mx8_fwd: need C = 128 and hidden a multiple of 128 (got %d, %d)",
                   a->C, a->hidden);
  if (a->rows <= 0) return pf_fail(PF_E_INVALID, "pf_transition_mx8_fwd: rows must be positive");
  if (!a->x_in || !a->out || !a->norm_w || !a->norm_b || !a->fc1_q || !a->fc1_s || !a->fc2_q || !a->fc2_s ||
      !a->fc3_q || !a->fc3_s)
    return pf_fail(PF_E_INVALID, "pf_transition_mx8_fwd: null pointer argument");
  const long waves = (a->rows + 31) / 32;
  const int grid = (int)((waves + 3) / 4);
  tr8_pair_kernel<false><<<grid, 256, 0, (hipStream_t)a->stream>>>(
      a->x_in, a->out, a->norm_w, a->norm_b, (const uint8_t*)a->fc1_q, (const uint8_t*)a->fc1_s,
      (const uint8_t*)a->fc2_q, (const uint8_t*)a->fc2_s, (const uint8_t*)a->fc3_q, (const uint8_t*)a->fc3_s,
      a->rows, a->hidden, a->accumulate, a->eps, ZBiasArgs{});
  PF_CHECK_LAUNCH("tr8_pair_kernel");
  return PF_OK;
}

extern "C" int pf_transition_mx8_pair_bias_fwd(const pf_transition_mx8_args* a, const pf_apb_args* apb) {
  if (!a || !apb) return pf_fail(PF_E_INVALID, "pf_transition_mx8_pair_bias_fwd: null args");
  if (a->C != C || a->hidden <= 0 || a->hidden % 128)
    return pf_fail(PF_E_INVALID,
                   "pf_transition_mx8_pair_bias_fwd: need C = 128 and hidden a multiple of 128 (got %d, %d)", a->C,
                   a->hidden);
  if (!a->x_in || !a->out || !a->norm_w || !a->norm_b || !a->fc1_q || !a->fc1_s || !a->fc2_q || !a->fc2_s ||
      !a->fc3_q || !a->fc3_s)
    return pf_fail(PF_E_INVALID, "pf_transition_mx8_pair_bias_fwd: null pointer argument");
  pf_apb_args chk = *apb;
  chk.z = a->out;   // the bias is computed from the transition's output
  int rc = pf_apb_check(&chk, "pf_transition_mx8_pair_bias_fwd", true);
  if (rc) return rc;
  const long NN = (long)apb->N * apb->N;
  if (a->rows != (long)apb->B * NN || a->rows % 128)
    return pf_fail(PF_E_INVALID, "pf_transition_mx8_pair_bias_fwd: rows %ld must equal B*N*N = %ld (a multiple of 128)",
                   a->rows, (long)apb->B * NN);
  const ZBiasArgs zb{apb->zln_w, apb->zln_b, (const op_t*)apb->w_z, pf_apb_bias_ptr(apb), NN, apb->H, apb->eps};
  tr8_pair_kernel<true><<<(unsigned)(a->rows / 128), 256, 0, (hipStream_t)a->stream>>>(
      a->x_in, a->out, a->norm_w, a->norm_b, (const uint8_t*)a->fc1_q, (const uint8_t*)a->fc1_s,
      (const uint8_t*)a->fc2_q, (const uint8_t*)a->fc2_s, (const uint8_t*)a->fc3_q, (const uint8_t*)a->fc3_s,
      a->rows, a->hidden, a->accumulate, a->eps, zb);
  PF_CHECK_LAUNCH("tr8_pair_kernel");
  return PF_OK;
}
