// Measurement aids for the benchmark: in-layer launch timing of chosen kernels (the
// triangle-attention core, the fp8 contraction), and the MFMA issue rate the chip sustains under
// load (its clock drops below the nameplate one when both MFMA pipes run on random operands).
#include <vector>

#include "pf_common.h"
#include "pf_internal.h"

namespace {

// Events bracketing every launch of one timed kernel kind (PF_TIMED_*) of this host thread
// while timing of that kind is on.  A pool grows to the largest count seen and is reused; it is
// never destroyed (a thread-local destructor would run after the HIP runtime is gone at process
// exit).
struct KernelTimer {
  bool on = false;
  size_t used = 0;
  int error = 0;
  std::vector<hipEvent_t> ev;   // begin, end, begin, end, ...
};
thread_local KernelTimer* g_timers[PF_TIMED_KINDS] = {};

KernelTimer* timer(int kind) {
  if (kind < 0 || kind >= PF_TIMED_KINDS) return nullptr;
  if (!g_timers[kind]) g_timers[kind] = new KernelTimer();
  return g_timers[kind];
}

}  // namespace

void pf_kernel_mark(int kind, hipStream_t st, int end) {
  KernelTimer* t = timer(kind);
  if (!t || !t->on || t->error) return;
  if ((t->used & 1) != (size_t)end) { t->error = 1; return; }   // unpaired mark
  if (t->used == t->ev.size()) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) { t->error = 1; return; }
    t->ev.push_back(e);
  }
  if (hipEventRecord(t->ev[t->used], st) != hipSuccess) { t->error = 1; return; }
  ++t->used;
}

void pf_attend_mark(hipStream_t st, int end) { pf_kernel_mark(PF_TIMED_ATTEND, st, end); }

extern "C" int pf_kernel_timing(int kind, int enable) {
  KernelTimer* t = timer(kind);
  if (!t) return pf_fail(PF_E_INVALID, "pf_kernel_timing: unknown kind %d", kind);
  t->on = enable != 0;
  if (t->on) {
    t->used = 0;
    t->error = 0;
  }
  return PF_OK;
}

extern "C" int pf_kernel_timing_read(int kind, double* total_ms, int* launches) {
  if (!total_ms || !launches) return pf_fail(PF_E_INVALID, "pf_kernel_timing_read: null output pointer");
  KernelTimer* t = timer(kind);
  if (!t) return pf_fail(PF_E_INVALID, "pf_kernel_timing_read: unknown kind %d", kind);
  if (t->error) return pf_fail(PF_E_LAUNCH, "pf_kernel_timing_read: an event could not be created or recorded");
  *total_ms = 0.0;
  *launches = (int)(t->used / 2);
  if (t->used >= 2) {
    const hipError_t e = hipEventSynchronize(t->ev[t->used - 1]);
    if (e != hipSuccess) return pf_fail(PF_E_LAUNCH, "pf_kernel_timing_read: %s", hipGetErrorString(e));
  }
  for (size_t i = 0; i + 1 < t->used; i += 2) {
    float ms = 0.f;
    const hipError_t e = hipEventElapsedTime(&ms, t->ev[i], t->ev[i + 1]);
    if (e != hipSuccess) return pf_fail(PF_E_LAUNCH, "pf_kernel_timing_read: %s", hipGetErrorString(e));
    *total_ms += ms;
  }
  return PF_OK;
}

extern "C" int pf_attend_timing(int enable) { return pf_kernel_timing(PF_TIMED_ATTEND, enable); }

extern "C" int pf_attend_timing_read(double* total_ms, int* launches) {
  return pf_kernel_timing_read(PF_TIMED_ATTEND, total_ms, launches);
}

namespace {

// Back-to-back 32x32x16 MFMAs on four independent accumulators; the operands rotate through
// four pseudo-random fragments per side (values in (-1, 1)), so the multiplier inputs toggle
// as in a GEMM.  Every wave writes one float so nothing is dead code.
constexpr int PROBE_WAVES = 16;

PF_DEV uint32_t mix32(uint32_t x) {
  x ^= x >> 16; x *= 0x7feb352dU; x ^= x >> 15; x *= 0x846ca68bU; x ^= x >> 16;
  return x;
}

__global__ __launch_bounds__(64 * PROBE_WAVES) void mfma_rate_kernel(int iters, float* __restrict__ sink) {
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  opx8 a[4], b[4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const uint32_t ra = mix32(tid * 64 + u * 8 + t), rb = mix32(ra ^ 0x9e3779b9U);
      a[u][t] = (op_t)((float)(ra >> 8) * (2.f / 16777216.f) - 1.f);
      b[u][t] = (op_t)((float)(rb >> 8) * (2.f / 16777216.f) - 1.f);
    }
  f32x16 acc[4] = {zero16(), zero16(), zero16(), zero16()};
  // the rotation is unrolled so every operand index is a constant (registers, not scratch)
  for (int i = 0; i < iters; i += 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] = mfma32(a[(u + j) & 3], b[(u + 2 * j) & 3], acc[u]);
  }
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[u][r];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) sink[tid >> 6] = s;
}

// The same on the block-scaled fp8 MFMA (32x32x64, e4m3 operands, unit scales), two fragments
// per side (four would not fit in the 128 registers of four waves per SIMD): bytes with bit 6
// clear (exponent field below 8, never NaN) drawn per lane from the same hash; the operand
// pair still changes with every MFMA.
__global__ __launch_bounds__(64 * PROBE_WAVES) void mfma8_rate_kernel(int iters, float* __restrict__ sink) {
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  i32x8 a[2], b[2];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const uint32_t ra = mix32(tid * 64 + u * 8 + t), rb = mix32(ra ^ 0x9e3779b9U);
      a[u][t] = (int)(ra & 0xBFBFBFBFu);
      b[u][t] = (int)(rb & 0xBFBFBFBFu);
    }
  f32x16 acc[4] = {zero16(), zero16(), zero16(), zero16()};
  for (int i = 0; i < iters; i += 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] = mfma8(a[(u + j) & 1], b[((u >> 1) + j) & 1], acc[u], 127, 127);
  }
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[u][r];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) sink[tid >> 6] = s;
}

}  // namespace

extern "C" int pf_mfma8_rate_probe(int workgroups, int iters, float* sink, void* stream) {
  if (workgroups <= 0 || iters <= 0 || iters % 4 || !sink)
    return pf_fail(PF_E_INVALID, "pf_mfma8_rate_probe: need workgroups > 0, iters > 0 a multiple of 4 and a sink "
                   "of workgroups * %d floats (got %d, %d, %p)", PROBE_WAVES, workgroups, iters, (void*)sink);
  mfma8_rate_kernel<<<workgroups, 64 * PROBE_WAVES, 0, (hipStream_t)stream>>>(iters, sink);
  PF_CHECK_LAUNCH("mfma8_rate_kernel");
  return PF_OK;
}

extern "C" long pf_mfma_rate_probe_waves(int workgroups) {
  return workgroups > 0 ? (long)workgroups * PROBE_WAVES : 0;
}

extern "C" int pf_mfma_rate_probe(int workgroups, int iters, float* sink, void* stream) {
  if (workgroups <= 0 || iters <= 0 || iters % 4 || !sink)
    return pf_fail(PF_E_INVALID, "pf_mfma_rate_probe: need workgroups > 0, iters > 0 a multiple of 4 and a sink "
                   "of workgroups * %d floats (got %d, %d, %p)", PROBE_WAVES, workgroups, iters, (void*)sink);
  mfma_rate_kernel<<<workgroups, 64 * PROBE_WAVES, 0, (hipStream_t)stream>>>(iters, sink);
  PF_CHECK_LAUNCH("mfma_rate_kernel");
  return PF_OK;
}
