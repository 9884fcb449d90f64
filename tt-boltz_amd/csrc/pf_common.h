// Shared device helpers for the Pairformer CDNA4 (gfx950) kernels.
//
// Operand type.  MFMA operands (weights, normalized activations, attention Q/K/V/P,
// trimul a/b planes) are `op_t`: IEEE fp16 by default, bf16 when built with
// -DPF_OPERAND_BF16.  On gfx950 both run at the same dense MFMA rate; fp16 carries
// 3 more mantissa bits, which is what keeps the bf16-class kernels inside the fp32
// parity bar.  Accumulation, LayerNorm/softmax statistics and the residual stream
// are fp32 in both builds.
//
// MFMA conventions used by every kernel in this library (wave64, fp32 acc):
//
//   v_mfma_f32_32x32x16_{f16,bf16}   D[32x32] += A[32x16] * B[16x32]
//     A operand  lane l: row    m = l & 31, k = 8*(l >> 5) + t   (t = 0..7, one opx8)
//     B operand  lane l: column n = l & 31, k = 8*(l >> 5) + t
//     C/D        lane l, reg r (0..15): column n = l & 31,
//                                      row    m = 8*(r >> 2) + 4*(l >> 5) + (r & 3)
//
// A GEMM only needs A and B to agree on which (lane half, slot) carries which k, so
// a "k permutation" applied to both operands leaves the product unchanged.  Kernels
// use this to feed an accumulator straight back in as the next MFMA's A/B operand:
// accumulator regs 8*s .. 8*s+7 of a lane in half h hold rows
//   16*s + 4*h + {0,1,2,3}  and  16*s + 8 + 4*h + {0,1,2,3}
// so the partner operand is loaded with the same two 4-element runs (kperm_row()),
// or the producer's rows are pre-permuted so the runs come out contiguous (perm16()).
#pragma once
#include <hip/hip_runtime.h>
#include <type_traits>
#include <stdint.h>

#ifdef PF_OPERAND_BF16
typedef __bf16 op_t;
#else
typedef _Float16 op_t;
#endif
typedef op_t opx8 __attribute__((ext_vector_type(8)));
typedef op_t opx4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define PF_DEV __device__ __forceinline__
// Device lambdas: always inlined (an outlined lambda moves captured state through memory).
#define PF_INLINE __attribute__((always_inline))

PF_DEV f32x16 mfma32(const opx8& a, const opx8& b, const f32x16& c) {
#ifdef PF_OPERAND_BF16
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
#else
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
#endif
}

PF_DEV f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Row of the 32x32 accumulator held by register r of a lane in half h.
PF_DEV int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// k index carried by slot t (0..7) of a lane in half h for k-step s when the
// operand comes from accumulator registers 8*s .. 8*s+7 (see header comment).
PF_DEV int kperm_row(int s, int h, int t) { return 16 * s + 4 * h + (t < 4 ? t : t + 4); }

// Involution on row indices swapping bits 2 and 3.  If a producer GEMM's weight row
// rho holds output unit perm16(rho), accumulator regs 8*s+t of half h come out as
// units 16*s + 8*h + t: the natural k order of the next MFMA operand.
PF_DEV int perm16(int row) { return (row & ~0xC) | ((row & 4) << 1) | ((row & 8) >> 1); }

PF_DEV float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }   // v_exp_f32

// v_rcp_f32 (1 ulp) instead of the IEEE division sequence HIP emits for '/'.
PF_DEV float rcp_fast(float x) { return __builtin_amdgcn_rcpf(x); }

// compile-time index for unrolled, stage-selected lambdas
template <int V>
using ic = std::integral_constant<int, V>;

// sigmoid(x) = 1 / (1 + 2^(-x log2 e)): saturates cleanly to 0 / 1 for large |x|.
PF_DEV float sigmoidf_fast(float x) { return rcp_fast(1.f + exp2_fast(-1.4426950408889634f * x)); }

PF_DEV float siluf(float x) { return x * sigmoidf_fast(x); }

// Sum / maximum over the lane pair (n, n + 32) of a wave64.  (A v_permlane32_swap form
// avoids the LDS round trip of ds_bpermute but measured slower in tm_out_kernel: +8-10 us
// at N = 512, the other pair kernels unchanged.)
PF_DEV float xor32_sum(float v) { return v + __shfl_xor(v, 32); }
PF_DEV float xor32_max(float v) { return fmaxf(v, __shfl_xor(v, 32)); }

// Full wave64 reductions.
PF_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
PF_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

PF_DEV opx8 ld_x8(const op_t* p) { return *reinterpret_cast<const opx8*>(p); }
PF_DEV opx4 ld_x4(const op_t* p) { return *reinterpret_cast<const opx4*>(p); }
PF_DEV void st_x8(op_t* p, const opx8& v) { *reinterpret_cast<opx8*>(p) = v; }
PF_DEV void st_x4(op_t* p, const opx4& v) { *reinterpret_cast<opx4*>(p) = v; }

PF_DEV opx8 cat44(const opx4& a, const opx4& b) {
  opx8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

PF_DEV opx8 zero_x8() {
  opx8 r;
#pragma unroll
  for (int t = 0; t < 8; ++t) r[t] = (op_t)0.f;
  return r;
}

// Load the x-hat fragment layout: lane (m = l & 31, h = l >> 5) reads channels
// 16*s + 8*h + t (s < CC/16, t = 0..7) of a CC-channel fp32 vector (CC = 64 or 128).
template <int CC>
PF_DEV void load_row_frag(const float* __restrict__ p, int h, float (&x)[CC / 2]) {
#pragma unroll
  for (int s = 0; s < CC / 16; ++s) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p + 16 * s + 8 * h);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 16 * s + 8 * h + 4);
    x[8 * s + 0] = a[0]; x[8 * s + 1] = a[1]; x[8 * s + 2] = a[2]; x[8 * s + 3] = a[3];
    x[8 * s + 4] = b[0]; x[8 * s + 5] = b[1]; x[8 * s + 6] = b[2]; x[8 * s + 7] = b[3];
  }
}
PF_DEV void load_row128_frag(const float* __restrict__ p, int h, float (&x)[64]) { load_row_frag<128>(p, h, x); }

// (x - mean) * rstd * gamma[c] of a CC-vector (load_row_frag order: x[8 s + t] is channel
// 16 s + 8 h + t) as CC/16 MFMA fragments: the LayerNorm without beta, for callers that add
// W beta to the product in fp32 (gamma stays on the activation side, so the op_t weights are
// rounded once).  gamma may live in LDS.
template <int CC>
PF_DEV void ln_gamma_to_frag(const float (&x)[CC / 2], int h, const float* gamma, float eps, opx8 (&f)[CC / 16]) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CC / 2; ++i) s += x[i];
  const float mean = xor32_sum(s) * (1.f / CC);
  float v = 0.f;
#pragma unroll
  for (int i = 0; i < CC / 2; ++i) { const float d = x[i] - mean; v += d * d; }
  const float rstd = rsqrtf(xor32_sum(v) * (1.f / CC) + eps);
#pragma unroll
  for (int s8 = 0; s8 < CC / 16; ++s8) {
    const f32x4 g0 = *reinterpret_cast<const f32x4*>(gamma + 16 * s8 + 8 * h);
    const f32x4 g1 = *reinterpret_cast<const f32x4*>(gamma + 16 * s8 + 8 * h + 4);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      f[s8][t] = (op_t)((x[8 * s8 + t] - mean) * (rstd * g0[t]));
      f[s8][4 + t] = (op_t)((x[8 * s8 + 4 + t] - mean) * (rstd * g1[t]));
    }
  }
}

// (x - mean) * rstd of a CC-vector (load_row_frag order) as CC/16 MFMA fragments: the
// LayerNorm without its affine part, for callers that fold gamma / beta into the weights.
template <int CC>
PF_DEV void ln_norm_to_frag(const float (&x)[CC / 2], float eps, opx8 (&f)[CC / 16]) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CC / 2; ++i) s += x[i];
  const float mean = xor32_sum(s) * (1.f / CC);
  float v = 0.f;
#pragma unroll
  for (int i = 0; i < CC / 2; ++i) { const float d = x[i] - mean; v += d * d; }
  const float rstd = rsqrtf(xor32_sum(v) * (1.f / CC) + eps);
#pragma unroll
  for (int s8 = 0; s8 < CC / 16; ++s8)
#pragma unroll
    for (int t = 0; t < 8; ++t) f[s8][t] = (op_t)((x[8 * s8 + t] - mean) * rstd);
}
PF_DEV void ln128_norm_to_frag(const float (&x)[64], float eps, opx8 (&f)[8]) { ln_norm_to_frag<128>(x, eps, f); }

// LayerNorm of a CC-vector split over the two halves of a wave (CC/2 values per
// lane, in load_row_frag order), written as CC/16 opx8 MFMA fragments.
// Two-pass (mean, then centred variance) in fp32, like torch's CPU kernel.
template <int CC>
PF_DEV void ln_to_frag(const float (&x)[CC / 2], int h, const float* __restrict__ w,
                       const float* __restrict__ b, float eps, opx8 (&f)[CC / 16]) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CC / 2; ++i) s += x[i];
  const float mean = xor32_sum(s) * (1.f / CC);
  float v = 0.f;
#pragma unroll
  for (int i = 0; i < CC / 2; ++i) { const float d = x[i] - mean; v += d * d; }
  const float rstd = rsqrtf(xor32_sum(v) * (1.f / CC) + eps);
#pragma unroll
  for (int s8 = 0; s8 < CC / 16; ++s8) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int c = 16 * s8 + 8 * h + t;
      f[s8][t] = (op_t)((x[8 * s8 + t] - mean) * rstd * w[c] + b[c]);
    }
  }
}
PF_DEV void ln128_to_frag(const float (&x)[64], int h, const float* __restrict__ w, const float* __restrict__ b,
                          float eps, opx8 (&f)[8]) {
  ln_to_frag<128>(x, h, w, b, eps, f);
}

// 16-byte-chunk XOR swizzle for LDS rows of 64 op_t (128 bytes): the 32 rows one
// MFMA operand read touches at one chunk index land on distinct bank groups.
PF_DEV int swz8r(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }

// LN over the 64 channels of a row held as channels 16 st + 8 h + t (st = 0..3) by lane
// half h, as 4 MFMA fragments.
PF_DEV void ln64_to_frag(const float* __restrict__ row, int h, const float* __restrict__ w,
                         const float* __restrict__ b, float eps, opx8 (&f)[4]) {
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
  const float mean = xor32_sum(sm) * (1.f / 64.f);
  float var = 0.f;
#pragma unroll
  for (int k = 0; k < 32; ++k) { const float d = x[k] - mean; var += d * d; }
  const float rstd = rsqrtf(xor32_sum(var) * (1.f / 64.f) + eps);
#pragma unroll
  for (int st = 0; st < 4; ++st)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int c = 16 * st + 8 * h + t;
      f[st][t] = (op_t)((x[8 * st + t] - mean) * rstd * w[c] + b[c]);
    }
}

// s_waitcnt immediate (gfx9 encoding) that waits until at most v vector-memory
// operations of this wave are outstanding and leaves expcnt / lgkmcnt unconstrained.
constexpr int vmcnt_le(int v) { return (v & 0xF) | (((v >> 4) & 3) << 14) | 0x70 | 0xF00; }

// 16-byte stores from the [d][pos] accumulator layout.  Lane (m, h) holds, for run g,
// the 4 values of elements 8g + 4h .. 8g + 4h + 3 (acc registers 4g .. 4g + 3).  One
// v_permlane32_swap per dword gives lane (m, 0) elements 8(2p+1) .. +7 and lane (m, 1)
// elements 16p .. 16p + 7 of run pair p, so each lane then writes 8 consecutive
// elements (16 bytes of op_t): half-row pieces of 16 bytes are half as fast to write.
// Writes elements [16p + 8(1-h), +8) of row `dst` (op_t, element 0 at dst) for p = 0, 1.
PF_DEV void store_runs16(op_t* dst, const f32x16& acc, float scale, int h) {
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    uint32_t u[2][2];   // [run 2p / 2p+1][dword]
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int dw = 0; dw < 2; ++dw) {
        typedef op_t pair_t __attribute__((ext_vector_type(2)));
        pair_t v;
        v[0] = (op_t)(acc[4 * (2 * p + k) + 2 * dw] * scale);
        v[1] = (op_t)(acc[4 * (2 * p + k) + 2 * dw + 1] * scale);
        u[k][dw] = __builtin_bit_cast(uint32_t, v);
      }
    uint32_t x[2], y[2];
#pragma unroll
    for (int dw = 0; dw < 2; ++dw) {
      const auto r = __builtin_amdgcn_permlane32_swap(u[1][dw], u[0][dw], false, false);
      x[dw] = r[0];   // lanes 0-31: own run 2p+1; lanes 32-63: run 2p of the lane 32 below
      y[dw] = r[1];   // lanes 0-31: run 2p+1 of the lane 32 above; lanes 32-63: own run 2p
    }
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    const u32x4_t v = {x[0], x[1], y[0], y[1]};
    *reinterpret_cast<u32x4_t*>(dst + 16 * p + 8 * (1 - h)) = v;
  }
}

// Decode of a wave-uniform tile index t (32 consecutive positions) of a [B][N][N] grid of
// positions, N % 32 == 0 and B * N * N < 2^32 (callers check on the host): batch b, row r,
// first column c0.  32-bit and uniform, so it is a short scalar sequence.
struct PosTile { int b, r, c0; };
PF_DEV PosTile pos_tile(uint32_t t, uint32_t N) {
  const uint32_t NN = N * N, pos0 = 32u * t;
  const uint32_t b = pos0 / NN, t0 = pos0 - b * NN, r = t0 / N;
  return {(int)b, (int)r, (int)(t0 - r * N)};
}

// Workgroup-id remap so that consecutive logical ids land on one XCD.
// Hardware dispatches workgroup w to XCD (w % 8); with total % 8 == 0 this maps
// the ids seen by XCD x to the contiguous range [x*total/8, (x+1)*total/8).
PF_DEV int xcd_remap(int w, int total) {
  if (total % 8) return w;
  return (w % 8) * (total / 8) + (w / 8);
}

// Fixed power-of-two scale of 16-bit contraction outputs X (the outer product mean's Z and
// the standalone contraction API): X is stored as X * 2^-8, so |X| up to ~1.7e7 fits fp16.
constexpr float X_STORE_SCALE = 1.f / 256.f;
constexpr float X_LOAD_SCALE = 256.f;

// Per-call power-of-two scale of the trimul contraction planes X = sum_k a_ik b_jk.  The
// producer of a and b leaves one max(|a|, |b|) per workgroup in `parts`; with amax the
// largest of them, |X| <= K * amax^2 =: f * 2^e (0.5 <= f < 1), and X is stored as
// X * 2^(15 - e), i.e. at most 2^15 in magnitude (fp16's largest value is ~2^16), whatever
// the scale of the weights: typical |X| then sits many binades above fp16's subnormal range.
// Wave-uniform; every wave reduces the (few hundred) maxima itself.
PF_DEV float planes_amax(const float* __restrict__ parts, int nparts) {
  const int lane = threadIdx.x & 63;
  float mx = 0.f;
  for (int i = lane; i < nparts; i += 64) mx = fmaxf(mx, parts[i]);
  return wave_max(mx);
}
PF_DEV float x_store_scale(float amax, int K) {
  const float bound = (float)K * amax * amax;
  if (!(bound > 0.f) || !(bound < 3.0e38f)) return 1.f;   // all-zero planes (or no bound): unscaled
  int e;
  (void)frexpf(bound, &e);
  // the exponent is capped so the scale and its inverse stay normal floats: planes whose
  // bound lies below 2^-111 (tiny but nonzero operands, possible with bf16) are stored at
  // most 2^126 times larger, not times inf
  return ldexpf(1.f, min(15 - e, 126));
}

// ---------------------------------------------------------------------------------
// MXFP8 (fast mode): OCP e4m3 elements with one E8M0 power-of-two scale per 32
// consecutive elements along the contraction axis.
//
//   v_mfma_scale_f32_32x32x64_f8f6f4 (cbsz = blgp = 0: e4m3 x e4m3), K = 64 per MFMA.
//   Operand lane l (row/column r = l & 31, half h = l >> 5) holds 32 bytes (8 dwords):
//     bytes  0..15  = elements 16h + (0..15)       of K block 0 (k  0..31)
//     bytes 16..31  = elements 16h + (0..15)       of K block 1 (k 32..63)
//   i.e. each 32-wide K block is split 16 + 16 between lanes r and r + 32, and the
//   block's scale byte is supplied by lane r + 32 * block (scale operand, byte 0).
//   A and B must agree on which (lane half, byte) carries which k; any permutation
//   inside a block applied to both operands leaves the product unchanged.
//   Accumulator layout as for the 16-bit MFMAs.
// Block scale: the smallest power of two X with amax / X <= 448, i.e. floor(log2(amax)) - 8
// (the OCP MX rule) plus one when amax's significand exceeds 1.75, so no element of a block
// is clamped (the plain OCP rule clamps block maxima in (448, 512) * X to 448).  Stored as
// the E8M0 byte log2(X) + 127 (0 for an all-zero block); elements round-to-nearest-even to
// e4m3 after division by X (the +-448 saturation is only a guard).
// ---------------------------------------------------------------------------------
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

PF_DEV f32x16 mfma8(const i32x8& a, const i32x8& b, const f32x16& c, int scale_a, int scale_b) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, scale_a, 0, scale_b);
}

// E8M0 scale byte of a block whose absolute maximum is amax (amax >= 0, finite): biased
// exponent of amax minus 8, one more when the significand is above 1.75 (fraction bits
// above 0x600000), clamped at 0 (covers amax == 0 and tiny blocks).
PF_DEV int mx_scale_byte(float amax) {
  const uint32_t u = __float_as_uint(amax);
  const int be = (int)((u >> 23) & 0xFF) + ((u & 0x7FFFFF) > 0x600000u ? 1 : 0);
  return max(be - 8, 0);
}

// 1 / X for a scale byte (X = 2^(byte - 127)): 2^(127 - byte), exact for byte 0..253.
PF_DEV float mx_inv_scale(int byte) { return __uint_as_float((uint32_t)(254 - byte) << 23); }

// Four floats (already divided by the block scale) -> four e4m3 bytes (value t in byte
// t), round to nearest even, saturating at +-448.
PF_DEV float sat448(float v) { return fminf(fmaxf(v, -448.f), 448.f); }
PF_DEV int e4m3_pack4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(a), sat448(b), 0, false);
  return __builtin_amdgcn_cvt_pk_fp8_f32(sat448(c), sat448(d), lo, true);
}

// 16 floats -> 4 dwords of e4m3 (element t in byte t), scaled by inv.
PF_DEV i32x4 e4m3_pack16(const float (&v)[16], float inv) {
  i32x4 r;
#pragma unroll
  for (int d = 0; d < 4; ++d)
    r[d] = e4m3_pack4(v[4 * d] * inv, v[4 * d + 1] * inv, v[4 * d + 2] * inv, v[4 * d + 3] * inv);
  return r;
}

PF_DEV i32x8 cat_i32x4(const i32x4& a, const i32x4& b) {
  i32x8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

PF_DEV float amax16(const float (&v)[16]) {
  float a = 0.f;
#pragma unroll
  for (int t = 0; t < 16; ++t) a = fmaxf(a, fabsf(v[t]));
  return a;
}

// ---------------------------------------------------------------------------------
// Quantize-dequantize ("fake quantization") in the format above, for values that stay in
// fp32 / op_t registers but must carry the block-fp8 rounding: v <- e4m3(v / X) * X.
// v_cvt_scalef32_pk_fp8_f32 divides by X and v_cvt_scalef32_pk_f32_fp8 multiplies by it,
// exactly (X is a power of two); neither saturates, which the scale rule makes unnecessary
// (|v / X| <= 448).  X is floored at 2^-126 (scale byte 1): only blocks whose maximum is
// below 2^-118 differ from the format's 2^-127, and all-zero blocks stay zero.
// ---------------------------------------------------------------------------------
typedef short i16x2 __attribute__((ext_vector_type(2)));

PF_DEV float mx_block_scale(float amax) { return __uint_as_float((uint32_t)max(mx_scale_byte(amax), 1) << 23); }

// One value with its own block scale X; `lim` = 448 X bounds v first (the block maximum
// was taken from a separately computed copy of the values, which may differ in the last bit).
PF_DEV float mx_fake_quant1(float v, float X, float lim) {
  const i16x2 w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(i16x2{0, 0}, __builtin_amdgcn_fmed3f(v, -lim, lim), 0.f,
                                                           X, false);
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(__builtin_bit_cast(int, w), X, false)[0];
}

// One 32-element block held as 16 values by each lane of the pair (n, n + 32), in place.
template <class V16>
PF_DEV void mx_fake_quant16(V16& v) {
  float a = 0.f;
#pragma unroll
  for (int t = 0; t < 16; ++t) a = fmaxf(a, fabsf(v[t]));
  const float X = mx_block_scale(xor32_max(a));
#pragma unroll
  for (int t = 0; t < 16; t += 2) {
    const i16x2 w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(i16x2{0, 0}, v[t], v[t + 1], X, false);
    const auto f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(__builtin_bit_cast(int, w), X, false);
    v[t] = f[0];
    v[t + 1] = f[1];
  }
}

// ---------------------------------------------------------------------------------
// "Output-aligned" layout of a 128-channel row for lane (position n, half h): the lane
// holds channels 32*(q>>2) + 8*(q&3) + 4h + e in x[4q + e] (chunk q = 0..15, e = 0..3),
// which are exactly the rows a 32x32 accumulator D[channel][position] (A = weight
// rows, B = activations) gives this lane for output block ob = q >> 2 in registers
// 4*(q&3) + e.  A residual update therefore adds x[16*ob + r] to accumulator register r
// of block ob, with no data exchange.  As an MFMA B operand, K step s (0..7) carries
// chunks 2s and 2s+1: slot t <-> channel 16s + 8*(t>>2) + 4h + (t&3); the weight
// (A operand) fragment of row m uses the same k order (wfrag_oa).
// ---------------------------------------------------------------------------------
PF_DEV int oa_channel(int q, int h) { return 32 * (q >> 2) + 8 * (q & 3) + 4 * h; }

template <int CC>
PF_DEV void load_row_oa(const float* __restrict__ p, int h, float (&x)[CC / 2]) {
#pragma unroll
  for (int q = 0; q < CC / 8; ++q) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p + oa_channel(q, h));
    x[4 * q + 0] = a[0]; x[4 * q + 1] = a[1]; x[4 * q + 2] = a[2]; x[4 * q + 3] = a[3];
  }
}

// (x - mean) * rstd * gamma[c] of a CC-channel row held in output-aligned order (x[4 q + e] is
// channel oa_channel(q, h) + e), as CC/16 MFMA B fragments: the LayerNorm without beta, for
// callers that add W beta in fp32 (the op_t weights stay rounded once).  gamma may live in LDS.
template <int CC>
PF_DEV void ln_oa_gamma_to_frag(const float (&x)[CC / 2], int h, const float* gamma, float eps,
                                opx8 (&f)[CC / 16]) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CC / 2; ++i) s += x[i];
  const float mean = xor32_sum(s) * (1.f / CC);
  float v = 0.f;
#pragma unroll
  for (int i = 0; i < CC / 2; ++i) { const float d = x[i] - mean; v += d * d; }
  const float rstd = rsqrtf(xor32_sum(v) * (1.f / CC) + eps);
#pragma unroll
  for (int q = 0; q < CC / 8; ++q) {
    const f32x4 g = *reinterpret_cast<const f32x4*>(gamma + oa_channel(q, h));
#pragma unroll
    for (int e = 0; e < 4; ++e) f[q >> 1][4 * (q & 1) + e] = (op_t)((x[4 * q + e] - mean) * (rstd * g[e]));
  }
}

// Weight fragment (A operand) of weight row `wrow` (128 op_t, contiguous) for K step s in
// the output-aligned k order.
PF_DEV opx8 wfrag_oa(const op_t* wrow, int s, int h) {
  return cat44(ld_x4(wrow + 16 * s + 4 * h), ld_x4(wrow + 16 * s + 8 + 4 * h));
}

// ---------------------------------------------------------------------------------
// Epilogue of the pair transitions (16-bit and block-fp8): out[p] = [out[p] +] update for the
// lane's pair p = pos0 + m, the update in the output-aligned layout (acc[ob][4g + e] is channel
// 32 ob + 8 g + 4 h + e).  ZBIAS: also the single-track pair bias of the updated row,
// bias[b][hd][i][j] = log2(e) * LN_zb(out[b,i,j,:]) . W_z[hd], from the values the lane has
// just written (no second pass over z); whole 32-pair tiles only.
// ---------------------------------------------------------------------------------
struct ZBiasArgs {
  const float* lnw; const float* lnb; const op_t* wz; float* bias;
  long NN; int H; float eps;
};

template <bool ZBIAS>
PF_DEV void pair_update_epilogue(const f32x16 (&acc)[4], float* out, long rows, long pos0, int m, int h,
                                 int accumulate, const ZBiasArgs& zb) {
  // lane (m, h) owns pair pos0 + m; acc[ob][4g + e] is channel 32 ob + 8 g + 4 h + e.  The
  // residual (x_in may alias out) is loaded in 16-byte runs, all before the first store.
  const long p = pos0 + m;
  if (!ZBIAS) {
    if (p < rows) {
      float* dst = out + p * 128;
      f32x4 res[16];
#pragma unroll
      for (int q = 0; q < 16; ++q)
        res[q] = accumulate ? *reinterpret_cast<const f32x4*>(dst + oa_channel(q, h)) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[q >> 2][4 * (q & 3) + e] + res[q][e];
        *reinterpret_cast<f32x4*>(dst + oa_channel(q, h)) = v;
      }
    }
    return;
  }
  // ZBIAS: whole tiles only (rows is a multiple of 32, checked on the host)
  float* dst = out + p * 128;
  __builtin_amdgcn_sched_barrier(0);
  float zv[64];   // residual, then the updated row, in output-aligned order (in place)
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const f32x4 r = accumulate ? *reinterpret_cast<const f32x4*>(dst + oa_channel(q, h)) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) zv[4 * q + e] = r[e];
  }
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      zv[4 * q + e] += acc[q >> 2][4 * (q & 3) + e];
      v[e] = zv[4 * q + e];
    }
    *reinterpret_cast<f32x4*>(dst + oa_channel(q, h)) = v;
  }
  opx8 zf[8];
  {
    float sm = 0.f;
#pragma unroll
    for (int i = 0; i < 64; ++i) sm += zv[i];
    const float mean = xor32_sum(sm) * (1.f / 128.f);
    float var = 0.f;
#pragma unroll
    for (int i = 0; i < 64; ++i) { const float d = zv[i] - mean; var += d * d; }
    const float rstd = rsqrtf(xor32_sum(var) * (1.f / 128.f) + zb.eps);
    // the affine parameters are read 8 channels at a time (the scheduling barrier keeps
    // their loads from being hoisted together, which would need 128 more registers)
#pragma unroll
    for (int q2 = 0; q2 < 8; ++q2) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int q = 2 * q2 + u, c0 = oa_channel(q, h);
        const f32x4 g4 = *reinterpret_cast<const f32x4*>(zb.lnw + c0);
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(zb.lnb + c0);
#pragma unroll
        for (int e = 0; e < 4; ++e) zf[q2][4 * u + e] = (op_t)((zv[4 * q + e] - mean) * rstd * g4[e] + b4[e]);
      }
    }
  }
  // D[head][pair]: weight row m from global memory (4 KB, cache-resident); lanes m >= H
  // repeat row H - 1 and their output rows (heads >= H) are not stored
  __builtin_amdgcn_sched_barrier(0);
  f32x16 hb = zero16();
  const op_t* wrow = zb.wz + min(m, zb.H - 1) * 128;
#pragma unroll
  for (int s2 = 0; s2 < 8; ++s2) hb = mfma32(wfrag_oa(wrow, s2, h), zf[s2], hb);
  // lane (pair m, h) holds heads acc_row(r, h); the tile's 32 pairs are consecutive (i, j)
  const long b = pos0 / zb.NN;
  float* brow = zb.bias + b * zb.H * zb.NN + (pos0 - b * zb.NN) + m;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int hd = acc_row(r, h);
    if (hd < zb.H) brow[hd * zb.NN] = hb[r] * 1.4426950408889634f;
  }
}

namespace {

// ---------------------------------------------------------------------------------
// Mean correction of the 16-bit input-side weights.  A weight W rounded to W16 makes the same
// error W_lo = W - W16 at every position; what survives a deep stack is its product with the
// mean of the normalized activation over positions.  The kernels therefore add, per output row,
// the fp32 offset  W . beta + W_lo . (gamma * mu),  mu = the mean over positions of the LayerNorm
// input normalized without its affine part (x_hat), and multiply the rounded activation by W16
// alone: the remaining error only meets the activation's deviation from its mean.
//   pair_stats_kernel  mu of z (batch 0) from PS_TILES tiles of 32 consecutive positions spread
//                      over the grid by Fibonacci hashing (every tile when there are fewer), as
//                      PS_WG partial sums already divided by the sample size
//   stats_mu           a workgroup sums the partials into mu (LDS) in its prologue
// ---------------------------------------------------------------------------------
#ifndef PF_PS_TILES
#define PF_PS_TILES 1024
#endif
// 64 workgroups of 16 waves, one tile per wave (at the default sample size)
constexpr int PS_WG = 64, PS_WAVES = 16, PS_TILES = PF_PS_TILES;
constexpr int PS_C = 128;   // channels of the pair rows the statistics are taken over
constexpr size_t PS_PARTIAL_FLOATS = (size_t)PS_WG * PS_C;

// v of the lane that the DPP control CTRL selects (within each row of 16 lanes)
template <int CTRL>
PF_DEV float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over each row of 16 lanes, left in every lane of the row: lane ^ 1, lane ^ 2 (quad
// permutes), then the other quad (row_half_mirror: i <-> 7 - i) and the other half-row
// (row_mirror: i <-> 15 - i).
PF_DEV float row16_sum(float v) {
  v += dpp_f<0xB1>(v);    // quad_perm [1, 0, 3, 2]
  v += dpp_f<0x4E>(v);    // quad_perm [2, 3, 0, 1]
  v += dpp_f<0x141>(v);   // row_half_mirror
  v += dpp_f<0x140>(v);   // row_mirror
  return v;
}

// A wave reads its tile fully coalesced: lane l handles row 4 p + (l >> 4) of each group p of
// four rows, channels 4 (l & 15) .. +3 and 64 + 4 (l & 15) .. +3 (so 16 lanes read a row's
// 512 bytes as two 256-byte runs), and takes the row's LayerNorm statistics with DPP sums over
// its row of 16 lanes.
__global__ __launch_bounds__(64 * PS_WAVES) void pair_stats_kernel(const float* __restrict__ z, int N, float eps,
                                                                   float* __restrict__ partials) {
  __shared__ float red[PS_WAVES][PS_C];
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, q = lane & 15, wid = tid >> 6;
  const uint32_t ntiles = (uint32_t)N * N / 32;
  const uint32_t ns = ntiles < (uint32_t)PS_TILES ? ntiles : (uint32_t)PS_TILES;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  for (uint32_t k = blockIdx.x * PS_WAVES + wid; k < ns; k += PS_WG * PS_WAVES) {
    const uint32_t t = ns == ntiles ? k : (uint32_t)(((uint64_t)k * 2654435761ull) % ntiles);
    const float* tile = z + (size_t)t * 32 * PS_C + g * PS_C + 4 * q;
    float4 x[16];   // [2 p]: channels 4 q .., [2 p + 1]: channels 64 + 4 q .., of row 4 p + g
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      x[2 * p] = *reinterpret_cast<const float4*>(tile + 4 * p * PS_C);
      x[2 * p + 1] = *reinterpret_cast<const float4*>(tile + 4 * p * PS_C + 64);
    }
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const float4 a = x[2 * p], b = x[2 * p + 1];
      const float mean = row16_sum((a.x + a.y) + (a.z + a.w) + (b.x + b.y) + (b.z + b.w)) * (1.f / PS_C);
      const float d[8] = {a.x - mean, a.y - mean, a.z - mean, a.w - mean,
                          b.x - mean, b.y - mean, b.z - mean, b.w - mean};
      float v = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) v += d[i] * d[i];
      const float rstd = rsqrtf(row16_sum(v) * (1.f / PS_C) + eps);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += d[i] * rstd;
    }
  }
  // the four lanes of a channel quad (g = 0..3) hold partial sums of the same channels
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    acc[i] += __shfl_xor(acc[i], 16);
    acc[i] += __shfl_xor(acc[i], 32);
  }
  if (lane < 16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      red[wid][4 * q + i] = acc[i];
      red[wid][64 + 4 * q + i] = acc[4 + i];
    }
  }
  __syncthreads();
  if (tid < PS_C) {
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < PS_WAVES; ++w) sum += red[w][tid];
    partials[blockIdx.x * PS_C + tid] = ns ? sum / (32.f * (float)ns) : 0.f;   // no tile: no correction
  }
}

// mu[c] (LDS, 128 floats) = the sum of the PS_WG partials, with every thread of the workgroup
// (blockDim.x a multiple of 128) summing a share into `scratch` (LDS, blockDim.x floats) first;
// the caller synchronizes before reading mu.
PF_DEV void stats_mu(const float* __restrict__ partials, float* mu, float* scratch) {
  const int nq = blockDim.x / PS_C, c = threadIdx.x % PS_C, q = threadIdx.x / PS_C;
  float sum = 0.f;
#pragma unroll 4
  for (int g = q; g < PS_WG; g += nq) sum += partials[g * PS_C + c];
  scratch[threadIdx.x] = sum;
  __syncthreads();
  if (threadIdx.x < PS_C) {
    float t = 0.f;
    for (int j = 0; j < nq; ++j) t += scratch[j * PS_C + threadIdx.x];
    mu[threadIdx.x] = t;
  }
}

// Prologue helpers of the persistent pair kernels.  Every global load of a thread's share is
// issued before the first use, so the set-up costs about one memory round trip instead of one
// per (partly unrolled) loop step; the arithmetic and its order are those of stats_mu,
// corrected_offset and a plain staging loop.
template <int NT>
constexpr int stats_per() { return PS_WG / (NT / PS_C); }
// this thread's partials (channel threadIdx.x % 128, groups q, q + NT / 128, ...)
template <int NT>
PF_DEV void stats_load(const float* __restrict__ partials, float (&v)[stats_per<NT>()]) {
  static_assert(NT % PS_C == 0 && PS_WG % (NT / PS_C) == 0, "block size");
  constexpr int nq = NT / PS_C;
  const int c = threadIdx.x % PS_C, q = threadIdx.x / PS_C;
#pragma unroll
  for (int i = 0; i < stats_per<NT>(); ++i) v[i] = partials[(q + i * nq) * PS_C + c];
}
// mu (LDS, 128 floats) from the loaded partials as stats_mu forms it; `scratch`: NT floats of
// LDS.  Synchronizes once; the caller synchronizes again before reading mu.
template <int NT>
PF_DEV void stats_reduce(const float (&v)[stats_per<NT>()], float* mu, float* scratch) {
  constexpr int nq = NT / PS_C;
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < stats_per<NT>(); ++i) sum += v[i];
  scratch[threadIdx.x] = sum;
  __syncthreads();
  if (threadIdx.x < PS_C) {
    float t = 0.f;
    for (int j = 0; j < nq; ++j) t += scratch[j * PS_C + threadIdx.x];
    mu[threadIdx.x] = t;
  }
}
// a 128-element op_t row in registers
PF_DEV void load_row_x8(const op_t* __restrict__ row, opx8 (&v)[PS_C / 8]) {
#pragma unroll
  for (int c = 0; c < PS_C / 8; ++c) v[c] = ld_x8(row + 8 * c);
}
// corrected_offset with the residual row already in registers (has_lo false: no correction);
// GAMMA false: no gamma factor (corrected_offset's gamma = nullptr: the product by 1 it takes is
// exact).  The LDS reads of gamma and mu go in groups of four chunks, so they are not all hoisted
// into registers at once.
template <bool GAMMA>
PF_DEV float corrected_offset_regs(float offb, const opx8 (&lo)[PS_C / 8], bool has_lo, const float* gamma,
                                   const float* mu) {
  float acc = offb;
  if (has_lo) {
#pragma unroll
    for (int c = 0; c < PS_C / 8; ++c) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float l = (float)lo[c][e];
        acc += (GAMMA ? l * gamma[8 * c + e] : l) * mu[8 * c + e];
      }
      if (c % 4 == 3) __builtin_amdgcn_sched_barrier(0);
    }
  }
  return acc;
}
// [ROWS][COLS] op_t weights: this thread's 16-byte chunks (chunk threadIdx.x + NT i), loaded
// all at once, then stored to LDS rows `pitch` elements apart (8-byte aligned rows: two 8-byte
// stores per chunk)
template <int NT, int ROWS, int COLS>
constexpr int stage_per() { return (ROWS * (COLS / 8) + NT - 1) / NT; }
template <int NT, int ROWS, int COLS>
PF_DEV void stage_load(const op_t* __restrict__ src, opx8 (&v)[stage_per<NT, ROWS, COLS>()]) {
  constexpr int CH = ROWS * (COLS / 8);
#pragma unroll
  for (int i = 0; i < stage_per<NT, ROWS, COLS>(); ++i) {
    const int c = threadIdx.x + NT * i;
    if (CH % NT == 0 || c < CH) v[i] = ld_x8(src + (c / (COLS / 8)) * COLS + (c % (COLS / 8)) * 8);
  }
}
template <int NT, int ROWS, int COLS>
PF_DEV void stage_store(op_t* dst, int pitch, const opx8 (&v)[stage_per<NT, ROWS, COLS>()]) {
  constexpr int CH = ROWS * (COLS / 8);
#pragma unroll
  for (int i = 0; i < stage_per<NT, ROWS, COLS>(); ++i) {
    const int c = threadIdx.x + NT * i;
    if (CH % NT == 0 || c < CH) {
      op_t* d = dst + (c / (COLS / 8)) * pitch + (c % (COLS / 8)) * 8;
      *reinterpret_cast<opx4*>(d) = opx4{v[i][0], v[i][1], v[i][2], v[i][3]};
      *reinterpret_cast<opx4*>(d + 4) = opx4{v[i][4], v[i][5], v[i][6], v[i][7]};
    }
  }
}

// Offset of one output row: offb (the fp32 W . beta) plus, with the mean correction, the row of
// the weight residual against gamma * mu (gamma, mu: 128 floats, LDS or global; gamma = nullptr
// when the kernel folds gamma into its weights, whose residual then already carries it).
PF_DEV float corrected_offset(float offb, const op_t* __restrict__ lo_row, const float* gamma, const float* mu) {
  float acc = offb;
  if (lo_row) {
#pragma unroll 4
    for (int c = 0; c < PS_C; c += 8) {
      const opx8 l8 = ld_x8(lo_row + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += (float)l8[e] * (gamma ? gamma[c + e] : 1.f) * mu[c + e];
    }
  }
  return acc;
}

}  // namespace
