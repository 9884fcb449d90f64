// Transition (SwiGLU MLP) and row primitives for gfx950.
//
//   tr_pair_kernel   Pair transition, C = 128: LN -> fc1|fc2 (MFMA, transposed
//                    orientation) -> silu(a)*b in registers -> fc3 (MFMA) -> residual.
//                    The 4C hidden activations never leave the CU.  fc1/fc2 rows are
//                    staged in LDS perm16-permuted so the fc1/fc2 accumulator registers
//                    come out in the natural k order of fc3's B operand.  Everything is in
//                    the output-aligned layout (pf_common.h): fc3 yields D[channel][pair],
//                    so a lane owns one pair and writes 16-byte runs, and the residual is
//                    fetched with 16-byte loads, all issued before the first store.  A wave
//                    owns PB*32 pairs so every weight fragment read from LDS feeds PB MFMAs.
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

// Launch configuration of the pair transition (pair blocks per wave, waves per WG,
// min waves per SIMD), chosen by measurement.
#ifndef TR_PB
#define TR_PB 1
#define TR_NW 4
#define TR_MINW 2
#endif

// PB: 32-pair blocks per wave; NW: waves per workgroup; MINW: min waves per SIMD hint.
template <int PB, int NW, int MINW>
__global__ __launch_bounds__(64 * NW, MINW) void tr_pair_kernel(
    const float* x_in, float* out, const float* __restrict__ lnw, const float* __restrict__ lnb,
    const op_t* __restrict__ w1, const op_t* __restrict__ w2, const op_t* __restrict__ w3,
    long rows, int hidden, int accumulate, float eps) {
  constexpr int NT = 64 * NW;            // threads
  constexpr int CH = 512 / NT;           // 16-byte chunks per thread per 8 KB block
  static_assert(NT <= 512 && 512 % NT == 0, "staging assumes 64..512 threads");
  __shared__ __attribute__((aligned(16))) op_t s1[2][32 * LDSW];
  __shared__ __attribute__((aligned(16))) op_t s2[2][32 * LDSW];
  __shared__ __attribute__((aligned(16))) op_t s3[2][C * LDS3];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, h = lane >> 5, m = lane & 31;
  const long pos0 = ((long)blockIdx.x * NW + wid) * (32 * PB);

  // Every wave runs the whole loop (no divergent control flow around the MFMA chain,
  // which would make the compiler shuttle accumulators between AGPRs and VGPRs);
  // rows past the end are clamped on load and skipped on store.
  opx8 xf[PB][8];
#pragma unroll
  for (int pb = 0; pb < PB; ++pb) {
    float x[64];
    load_row128_oa(x_in + min(pos0 + 32 * pb + m, rows - 1) * C, h, x);
    ln128_oa_to_frag(x, h, lnw, lnb, eps, xf[pb]);
  }
  f32x16 acc[PB][4];
#pragma unroll
  for (int pb = 0; pb < PB; ++pb)
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) acc[pb][ob] = zero16();

  // staging: fc1/fc2 block = 32 rows x 128, fc3 block = 128 rows x 32 (512 chunks each)
  opx8 r1[CH], r2[CH], r3[CH];
  auto gload = [&](int hb) {
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      const int c = tid + NT * q;
      r1[q] = ld_x8(w1 + (long)(32 * hb + (c >> 4)) * C + (c & 15) * 8);
      r2[q] = ld_x8(w2 + (long)(32 * hb + (c >> 4)) * C + (c & 15) * 8);
      r3[q] = ld_x8(w3 + (long)(c >> 2) * hidden + 32 * hb + (c & 3) * 8);
    }
  };
  const int nhb = hidden / 32;
  gload(0);
  for (int hb = 0; hb < nhb; ++hb) {
    const int bufi = hb & 1;
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      const int c = tid + NT * q;
      const int row = perm16(c >> 4);
      st_x8(&s1[bufi][row * LDSW + (c & 15) * 8], r1[q]);
      st_x8(&s2[bufi][row * LDSW + (c & 15) * 8], r2[q]);
      st_x8(&s3[bufi][(c >> 2) * LDS3 + (c & 3) * 8], r3[q]);
    }
    __syncthreads();
    if (hb + 1 < nhb) gload(hb + 1);
    f32x16 a1[PB], a2[PB];
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) { a1[pb] = zero16(); a2[pb] = zero16(); }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const opx8 f1 = wfrag_oa(&s1[bufi][m * LDSW], s, h);
      const opx8 f2 = wfrag_oa(&s2[bufi][m * LDSW], s, h);
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) {
        a1[pb] = mfma32(f1, xf[pb][s], a1[pb]);   // rows = hidden (perm16), cols = pairs
        a2[pb] = mfma32(f2, xf[pb][s], a2[pb]);
      }
    }
    opx8 hf[PB][2];
#pragma unroll
    for (int pb = 0; pb < PB; ++pb)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int t = 0; t < 8; ++t) hf[pb][ks][t] = (op_t)(siluf(a1[pb][8 * ks + t]) * a2[pb][8 * ks + t]);
#pragma unroll
    for (int ob = 0; ob < 4; ++ob)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const opx8 f3 = ld_x8(&s3[bufi][(32 * ob + m) * LDS3 + 16 * ks + 8 * h]);
#pragma unroll
        for (int pb = 0; pb < PB; ++pb) acc[pb][ob] = mfma32(f3, hf[pb][ks], acc[pb][ob]);   // D[ch][pair]
      }
  }
  // lane (m, h) owns pair pos0 + 32 pb + m; acc[pb][ob][4g + e] is channel 32 ob + 8 g + 4 h + e
#pragma unroll
  for (int pb = 0; pb < PB; ++pb) {
    const long p = pos0 + 32 * pb + m;
    if (p < rows) {
      float* dst = out + p * C;
      f32x4 res[16];
#pragma unroll
      for (int q = 0; q < 16; ++q)
        res[q] = accumulate ? *reinterpret_cast<const f32x4*>(dst + oa_channel(q, h)) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[pb][q >> 2][4 * (q & 3) + e] + res[q][e];
        *reinterpret_cast<f32x4*>(dst + oa_channel(q, h)) = v;
      }
    }
  }
}

// One wave per row.
__global__ __launch_bounds__(256) void ln_rows_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      const float* __restrict__ b, float* __restrict__ out,
                                                      long rows, int C_, float eps) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + row * C_;
  float s = 0.f;
  for (int c = lane; c < C_; c += 64) s += xr[c];
  const float mean = wave_sum(s) / C_;
  float v = 0.f;
  for (int c = lane; c < C_; c += 64) { const float d = xr[c] - mean; v += d * d; }
  const float rstd = rsqrtf(wave_sum(v) / C_ + eps);
  for (int c = lane; c < C_; c += 64) out[row * C_ + c] = (xr[c] - mean) * rstd * w[c] + b[c];
}

// One wave = 32 rows x 32 output columns; a workgroup = 4 waves along the columns.
// SWIGLU: out[:, n] = silu(x W[n]) * (x W2[n]).
template <bool SWIGLU>
__global__ __launch_bounds__(256) void linear_rows_kernel(
    const float* __restrict__ x, const op_t* __restrict__ W, const op_t* __restrict__ W2,
    const float* __restrict__ bias, const float* resid, float* out, long rows, int K, int Nout) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, h = lane >> 5, m = lane & 31;
  const int nt = blockIdx.y * 4 + wid;   // column tile
  if (nt * 32 >= Nout) return;
  const long r0 = (long)blockIdx.x * 32;
  const float* xr = x + min(r0 + m, rows - 1) * K;
  const op_t* wr = W + (long)(nt * 32 + m) * K;
  const op_t* wr2 = SWIGLU ? W2 + (long)(nt * 32 + m) * K : nullptr;
  f32x16 acc = zero16(), acc2 = zero16();
  for (int k0 = 0; k0 < K; k0 += 16) {
    const f32x4 a0 = *reinterpret_cast<const f32x4*>(xr + k0 + 8 * h);
    const f32x4 a1 = *reinterpret_cast<const f32x4*>(xr + k0 + 8 * h + 4);
    opx8 af;
    af[0] = (op_t)a0[0]; af[1] = (op_t)a0[1]; af[2] = (op_t)a0[2]; af[3] = (op_t)a0[3];
    af[4] = (op_t)a1[0]; af[5] = (op_t)a1[1]; af[6] = (op_t)a1[2]; af[7] = (op_t)a1[3];
    acc = mfma32(af, ld_x8(wr + k0 + 8 * h), acc);
    if (SWIGLU) acc2 = mfma32(af, ld_x8(wr2 + k0 + 8 * h), acc2);
  }
  const int n = nt * 32 + m;
  const float bn = bias ? bias[n] : 0.f;
  // residuals first (resid may alias out: all loads ahead of the stores, so they overlap)
  float res[16];
#pragma unroll
  for (int r = 0; r < 16; ++r)
    res[r] = !SWIGLU && resid ? resid[min(r0 + acc_row(r, h), rows - 1) * Nout + n] : 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const long row = r0 + acc_row(r, h);
    if (row >= rows) continue;
    out[row * Nout + n] = SWIGLU ? siluf(acc[r]) * acc2[r] : acc[r] + bn + res[r];
  }
}

// out[p, :] = base[p, :] + W . LN(x[p, :]),  C = 128; W resident in LDS.
__global__ __launch_bounds__(256) void pair_ln_linear_kernel(
    const float* x, const float* base, const float* __restrict__ lnw, const float* __restrict__ lnb,
    const op_t* __restrict__ W, float* out, long rows, float eps) {
  __shared__ __attribute__((aligned(16))) op_t sW[C * LDSW];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, h = lane >> 5, m = lane & 31;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int c = tid + 256 * q;
    st_x8(&sW[(c >> 4) * LDSW + (c & 15) * 8], ld_x8(W + (c >> 4) * C + (c & 15) * 8));
  }
  __syncthreads();
  const long pos0 = ((long)blockIdx.x * 4 + wid) * 32;
  if (pos0 >= rows) return;
  float xv[64];
  opx8 xf[8];
  load_row128_frag(x + min(pos0 + m, rows - 1) * C, h, xv);
  ln128_to_frag(xv, h, lnw, lnb, eps, xf);
#pragma unroll
  for (int ob = 0; ob < 4; ++ob) {
    f32x16 acc = zero16();
#pragma unroll
    for (int s = 0; s < 8; ++s) acc = mfma32(xf[s], ld_x8(&sW[(32 * ob + m) * LDSW + 16 * s + 8 * h]), acc);
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

static int launch_linear(const float* x, const void* W, const void* W2, const float* bias, const float* resid,
                         float* out, long rows, int K, int Nout, hipStream_t st) {
  if (!x || !W || !out) return pf_fail(PF_E_INVALID, "pf_linear_fwd: null pointer");
  if (rows <= 0 || K <= 0 || K % 16 || Nout <= 0 || Nout % 32)
    return pf_fail(PF_E_INVALID, "pf_linear_fwd: need rows > 0, K %% 16 == 0, Nout %% 32 == 0 (rows=%ld K=%d Nout=%d)",
                   rows, K, Nout);
  dim3 grid((unsigned)((rows + 31) / 32), (unsigned)((Nout / 32 + 3) / 4));
  if (W2)
    linear_rows_kernel<true><<<grid, 256, 0, st>>>(x, (const op_t*)W, (const op_t*)W2, nullptr, nullptr, out, rows, K, Nout);
  else
    linear_rows_kernel<false><<<grid, 256, 0, st>>>(x, (const op_t*)W, nullptr, bias, resid, out, rows, K, Nout);
  PF_CHECK_LAUNCH("linear_rows_kernel");
  return PF_OK;
}

extern "C" int pf_linear_fwd(const float* x, const void* W, const float* bias, const float* resid, float* out,
                             long rows, int K, int Nout, void* stream) {
  return launch_linear(x, W, nullptr, bias, resid, out, rows, K, Nout, (hipStream_t)stream);
}

extern "C" size_t pf_transition_workspace_size(long rows, int C_, int hidden) {
  if (rows <= 0 || C_ <= 0 || hidden <= 0) return 0;
  if (C_ == C && hidden % 32 == 0) return 0;   // fused pair kernel: no scratch
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
  if (a->C == C) {
    constexpr int PB = TR_PB, NW = TR_NW;
    const unsigned grid = (unsigned)((a->rows + 32 * PB * NW - 1) / (32 * PB * NW));
    tr_pair_kernel<PB, NW, TR_MINW><<<grid, 64 * NW, 0, st>>>(a->x_in, a->out, a->norm_w, a->norm_b, (const op_t*)a->fc1_w,
                                         (const op_t*)a->fc2_w, (const op_t*)a->fc3_w, a->rows, a->hidden,
                                         a->accumulate, a->eps);
    PF_CHECK_LAUNCH("tr_pair_kernel");
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
                                     const void* W, float* out, long rows, int C_, float eps, void* stream) {
  if (!x || !base || !ln_w || !ln_b || !W || !out) return pf_fail(PF_E_INVALID, "pf_pair_ln_linear_fwd: null pointer");
  if (C_ != C || rows <= 0) return pf_fail(PF_E_INVALID, "pf_pair_ln_linear_fwd: only C = 128 (got %d)", C_);
  pair_ln_linear_kernel<<<(unsigned)((rows + 127) / 128), 256, 0, (hipStream_t)stream>>>(
      x, base, ln_w, ln_b, (const op_t*)W, out, rows, eps);
  PF_CHECK_LAUNCH("pair_ln_linear_kernel");
  return PF_OK;
}
