// Diffusion conditioning, pair side, for gfx950: the two N^2-sized steps that run once
// per trunk output and stay fixed for every sampling step.
//
//   cond_proj_kernel   PairwiseConditioning's input projection (tt_bio/boltz2.py:1318-1355):
//                      out = W . LN(cat(z_trunk, rel_pos)) over 256 channels (LayerNorm with
//                      affine, folded into W as below; LinearNoBias 256 -> 128).  The two
//                      transitions that follow run on the pair transition kernel
//                      (transition.hip).
//   token_bias_kernel  DiffusionConditioning's token-transformer pair bias
//                      (tt_bio/boltz2.py:2434-2441, 2472-2475; the ttnn compute_bias of
//                      tt_bio/tenstorrent.py:714-728): for each of L layers,
//                      LN_l(z) . W_l^T (H heads, no bias), concatenated over layers.  All
//                      layers normalise the same z, so the statistics are computed once and
//                      each layer's affine is folded into its weights when they are staged:
//                      W'_l = W_l diag(gamma_l), b'_l = W_l beta_l.
//
// Both kernels are persistent (one workgroup of 8 waves per CU, weights resident in LDS,
// rows of 256 bytes with 16-byte chunk c at slot c ^ (R & 15)) and walk tiles of 32 pairs
// per wave: the LayerNorm runs in registers on the lane's half row, and the MFMA
// orientation is chosen per output layout so that stores are long contiguous runs
// (D[output][pair] for pair-major rows of 128 channels and for output planes,
// D[pair][output] for the wide pair-major bias rows).
#include "pf_common.h"
#include "pf_internal.h"

namespace {

constexpr int C = 128;       // c_z
constexpr int DF_WAVES = 8;
constexpr int TB_MAX_OUT = 512;
constexpr int TB_WAVES = 12;   // token bias: three waves per SIMD (<= 168 VGPRs: no scratch spills)

PF_DEV int slot16(int R, int c) { return R * C + 8 * (c ^ (R & 15)); }

// -------------------------------------------------------------------------------------
// out[p, :] = W . LN(cat(z[p, :], r[p, :]))  (W [128][256], LN over 256 with affine)
//          = W' . LNhat(cat(z, r)) + b'
// -------------------------------------------------------------------------------------
__global__ __launch_bounds__(64 * DF_WAVES, 1) void cond_proj_kernel(
    const float* __restrict__ z, const float* __restrict__ r, const float* __restrict__ lnw,
    const float* __restrict__ lnb, const op_t* __restrict__ W, float* __restrict__ out, long rows, float eps) {
  // W split by input half: sw[0] = W[:, 0:128] (z channels), sw[1] = W[:, 128:256]
  // the LayerNorm affine is folded in: W' = W diag(gamma) (staged), b' = W beta
  __shared__ __attribute__((aligned(16))) op_t sw[2][C * C];
  __shared__ float sb[C];
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, m = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
#pragma unroll 4
  for (int c = tid; c < 2 * C * 16; c += 64 * DF_WAVES) {   // 128 rows x 32 chunks
    const int R = c >> 5, k = c & 31;
    const opx8 wv = ld_x8(W + R * 2 * C + 8 * k);
    opx8 o;
#pragma unroll
    for (int u = 0; u < 8; ++u) o[u] = (op_t)((float)wv[u] * lnw[8 * k + u]);
    st_x8(&sw[k >> 4][slot16(R, k & 15)], o);
  }
#pragma unroll 4
  for (int R = wid; R < C; R += DF_WAVES) {   // one wave per output row, 4 channels per lane
    float v = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) v += (float)W[R * 2 * C + 64 * q + lane] * lnb[64 * q + lane];
    v = wave_sum(v);
    if (lane == 0) sb[R] = v;
  }
  __syncthreads();
  const long ntiles = (rows + 31) / 32;
  for (long t = (long)blockIdx.x * DF_WAVES + wid; t < ntiles; t += (long)gridDim.x * DF_WAVES) {
    const long p0 = 32 * t, row = min(p0 + m, rows - 1);
    opx8 xf[2][8];
    {
      float xz[64], xr[64];
      load_row128_frag(z + row * C, h, xz);
      load_row128_frag(r + row * C, h, xr);
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 64; ++i) s += xz[i] + xr[i];
      const float mean = xor32_sum(s) * (1.f / 256.f);
      float v = 0.f;
#pragma unroll
      for (int i = 0; i < 64; ++i) {
        const float a = xz[i] - mean, b = xr[i] - mean;
        v += a * a + b * b;
      }
      const float rstd = rsqrtf(xor32_sum(v) * (1.f / 256.f) + eps);
#pragma unroll
      for (int s8 = 0; s8 < 8; ++s8)
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          xf[0][s8][u] = (op_t)((xz[8 * s8 + u] - mean) * rstd);
          xf[1][s8][u] = (op_t)((xr[8 * s8 + u] - mean) * rstd);
        }
    }
    const bool live = p0 + m < rows;
    float* dst = out + (p0 + m) * C + 4 * h;
#pragma unroll 1
    for (int ob = 0; ob < 4; ++ob) {
      f32x16 acc = zero16();
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int s8 = 0; s8 < 8; ++s8)
          acc = mfma32(ld_x8(&sw[half][slot16(32 * ob + m, 2 * s8 + h)]), xf[half][s8], acc);
      // lane (pair m, h): acc[4 g + e] is output 32 ob + 8 g + 4 h + e
      if (live)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int o = 32 * ob + 8 * g + 4 * h;
          *reinterpret_cast<f32x4*>(dst + 32 * ob + 8 * g) =
              f32x4{acc[4 * g] + sb[o], acc[4 * g + 1] + sb[o + 1], acc[4 * g + 2] + sb[o + 2],
                    acc[4 * g + 3] + sb[o + 3]};
        }
    }
  }
}

// -------------------------------------------------------------------------------------
// bias[p, o] = scale * (W'[o] . LNhat(z[p]) + b'[o]),  o = l * H + hd < M
//   layout 0: out [rows][M]        (the reference's torch.cat(..., dim=-1) layout)
//   layout 1: out [M][rows]        (one contiguous [B][N][N] plane per (layer, head))
// -------------------------------------------------------------------------------------
__global__ __launch_bounds__(64 * TB_WAVES, 1) void token_bias_kernel(
    const float* __restrict__ z, const float* __restrict__ lnw, const float* __restrict__ lnb,
    const op_t* __restrict__ W, float* __restrict__ out, long rows, int M, int H, int layout, float scale,
    float eps) {
  __shared__ __attribute__((aligned(16))) op_t sw[TB_MAX_OUT * C];
  __shared__ float sb[TB_MAX_OUT];
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, m = lane & 31;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  // stage W'[o][c] = W[o][c] * gamma_l[c] (16 chunks of 8 channels per row)
#pragma unroll 4
  for (int c = tid; c < M * 16; c += 64 * TB_WAVES) {
    const int R = c >> 4, k = c & 15, l = R / H;
    const opx8 wv = ld_x8(W + R * C + 8 * k);
    opx8 o;
#pragma unroll
    for (int u = 0; u < 8; ++u) o[u] = (op_t)((float)wv[u] * lnw[l * C + 8 * k + u]);
    st_x8(&sw[slot16(R, k)], o);
  }
  // b'[o] = sum_c W[o][c] beta_l[c]: one wave per output row, two channels per lane
#pragma unroll 4
  for (int R = wid; R < M; R += TB_WAVES) {
    const int l = R / H;
    float v = (float)W[R * C + lane] * lnb[l * C + lane] + (float)W[R * C + 64 + lane] * lnb[l * C + 64 + lane];
    v = wave_sum(v);
    if (lane == 0) sb[R] = v;
  }
  __syncthreads();
  const long ntiles = (rows + 31) / 32;
  const int nob = M / 32;
  for (long t = (long)blockIdx.x * TB_WAVES + wid; t < ntiles; t += (long)gridDim.x * TB_WAVES) {
    const long p0 = 32 * t;
    const bool live = p0 + m < rows;
    opx8 xf[8];
    {
      float x[64];
      load_row128_frag(z + min(p0 + m, rows - 1) * C, h, x);
      ln128_norm_to_frag(x, eps, xf);
    }
    if (layout == 0) {
      // D[pair][output]: lane (output m, h) holds pairs acc_row(r, h), so each store
      // instruction writes two full 128-byte runs of one pair's row
#pragma unroll 1
      for (int ob = 0; ob < nob; ++ob) {
        f32x16 acc = zero16();
#pragma unroll
        for (int s8 = 0; s8 < 8; ++s8) acc = mfma32(xf[s8], ld_x8(&sw[slot16(32 * ob + m, 2 * s8 + h)]), acc);
        const float bo = sb[32 * ob + m];
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
          const long p = p0 + acc_row(rr, h);
          if (p < rows) out[p * M + 32 * ob + m] = scale * (acc[rr] + bo);
        }
      }
    } else {
      // D[output][pair]: lanes write 32 consecutive pairs of one output plane
#pragma unroll 1
      for (int ob = 0; ob < nob; ++ob) {
        f32x16 acc = zero16();
#pragma unroll
        for (int s8 = 0; s8 < 8; ++s8) acc = mfma32(ld_x8(&sw[slot16(32 * ob + m, 2 * s8 + h)]), xf[s8], acc);
        if (live)
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) {
            const int o = 32 * ob + acc_row(rr, h);
            out[(long)o * rows + p0 + m] = scale * (acc[rr] + sb[o]);
          }
      }
    }
  }
}

int launch_grid(long rows, int waves) {
  const int cus = device_cus();
  if (cus <= 0) return -1;
  const long tiles = (rows + 31) / 32;
  return (int)min((long)cus, (tiles + waves - 1) / waves);
}

}  // namespace

// ---------------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------------
extern "C" int pf_pair_cond_proj_fwd(const float* z, const float* rel_pos, const float* ln_w, const float* ln_b,
                                     const void* W, float* out, long rows, int c_z, float eps, void* stream) {
  if (!z || !rel_pos || !ln_w || !ln_b || !W || !out) return pf_fail(PF_E_INVALID, "pf_pair_cond_proj_fwd: null pointer");
  if (c_z != C || rows <= 0) return pf_fail(PF_E_INVALID, "pf_pair_cond_proj_fwd: need c_z = 128 and rows > 0 (got %d, %ld)", c_z, rows);
  if (out == z || out == rel_pos) return pf_fail(PF_E_INVALID, "pf_pair_cond_proj_fwd: out must not alias an input");
  const int grid = launch_grid(rows, DF_WAVES);
  if (grid <= 0) return pf_fail(PF_E_LAUNCH, "pf_pair_cond_proj_fwd: cannot query the device");
  cond_proj_kernel<<<grid, 64 * DF_WAVES, 0, (hipStream_t)stream>>>(z, rel_pos, ln_w, ln_b, (const op_t*)W, out, rows,
                                                                    eps);
  PF_CHECK_LAUNCH("cond_proj_kernel");
  return PF_OK;
}

extern "C" int pf_token_pair_bias_fwd(const float* z, const float* ln_w, const float* ln_b, const void* W, float* out,
                                      long rows, int c_z, int n_layers, int n_heads, int layout, float scale, float eps,
                                      void* stream) {
  if (!z || !ln_w || !ln_b || !W || !out) return pf_fail(PF_E_INVALID, "pf_token_pair_bias_fwd: null pointer");
  const long M = (long)n_layers * n_heads;
  if (c_z != C || rows <= 0 || n_layers <= 0 || n_heads <= 0 || M % 32 || M > TB_MAX_OUT || (layout != 0 && layout != 1))
    return pf_fail(PF_E_INVALID,
                   "pf_token_pair_bias_fwd: need c_z = 128, n_layers * n_heads a multiple of 32 up to %d, layout 0/1 "
                   "(got c_z=%d L=%d H=%d layout=%d rows=%ld)", TB_MAX_OUT, c_z, n_layers, n_heads, layout, rows);
  if (rows * M >= (1l << 40)) return pf_fail(PF_E_INVALID, "pf_token_pair_bias_fwd: shape too large");
  const int grid = launch_grid(rows, TB_WAVES);
  if (grid <= 0) return pf_fail(PF_E_LAUNCH, "pf_token_pair_bias_fwd: cannot query the device");
  token_bias_kernel<<<grid, 64 * TB_WAVES, 0, (hipStream_t)stream>>>(z, ln_w, ln_b, (const op_t*)W, out, rows, (int)M,
                                                                     n_heads, layout, scale, eps);
  PF_CHECK_LAUNCH("token_bias_kernel");
  return PF_OK;
}
