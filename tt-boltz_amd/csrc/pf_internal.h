// Host-side helpers shared by the C-ABI entry points (error reporting).
#pragma once
#include <hip/hip_runtime.h>
#include "pairformer_hip.h"

// Record a thread-local error message and return `code`.
int pf_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// After a launch: turn a launch error into PF_E_LAUNCH naming the kernel.
#define PF_CHECK_LAUNCH(name)                                                        \
  do {                                                                               \
    hipError_t e_ = hipGetLastError();                                               \
    if (e_ != hipSuccess)                                                            \
      return pf_fail(e_ == hipErrorOutOfMemory ? PF_E_OOM : PF_E_LAUNCH,             \
                     "%s launch failed: %s%s", name, hipGetErrorString(e_),          \
                     e_ == hipErrorOutOfMemory ? " (out of memory)" : "");           \
  } while (0)

// Compute units of the current device (cached per device; 0 if the query fails).
int device_cus();

// Allow `kernel` `bytes` of dynamic LDS on the current device.  The attribute is set once
// per (kernel, device), under a lock, and its status is kept: every later call on that
// device returns the same result (PF_OK, or PF_E_LAUNCH with the message set again).
int pf_reserve_lds(const void* kernel, size_t bytes, const char* name);

// One row-major projection out = resid + x W^T + bias (fp32 x/out, op_t W [Nout][K]);
// W2 != nullptr selects SwiGLU: out = silu(x W^T) * (x W2^T).  Up to PF_LIN_MAX_JOBS
// projections of one shape (rows, K, Nout) run in a single launch (transition.hip).
constexpr int PF_LIN_MAX_JOBS = 4;
struct pf_lin_job {
  const float* x;
  const void* W;
  const void* W2;
  const float* bias;
  const float* resid;
  float* out;
};
int pf_linear_batch(const pf_lin_job* jobs, int njobs, long rows, int K, int Nout, hipStream_t st);

// Single-track attention workspace helpers (single.hip): argument checks shared by the
// entry points (bias_only: only what the pair bias reads), and the address of the pair
// bias [B][H][N][N] inside the workspace.
int pf_apb_check(const pf_apb_args* a, const char* fn, bool bias_only, bool check_ws = true);
float* pf_apb_bias_ptr(const pf_apb_args* a);

// Batched X[p][i][j] = scale * sum_k A[p][i][k] * B[p][j][k] (trimul.hip): A [P][M][K],
// B [P][Nc][K] op_t, X [P][M][Nc] fp32 (x_fp32) or op_t; M, Nc % 32 == 0, K % 64 == 0.
int pf_contract_rect(const void* A, const void* B, void* X, int x_fp32, int planes, int M, int Nc, int K,
                     float scale, hipStream_t st);

// out[b][h][i][j] = log2(e) * LN(z[b,i,j,:]) . W_z[h] for H <= 32 heads, C = 128, B*N*N a
// multiple of 32 (single.hip: the single-track pair-bias kernel).
int pf_pair_logits(const float* z, const float* lnw, const float* lnb, const void* wz, float* out, int B, int N,
                   int H, float eps, hipStream_t st);

// Launch timing of the triangle-attention core (measure.hip): while pf_attend_timing(1) is on
// for this host thread, the launcher records an event before (end = 0) and after (end = 1)
// every ta_attn_kernel launch on its stream; otherwise a no-op.
void pf_attend_mark(hipStream_t st, int end);
// The same for any kind PF_TIMED_* (pf_kernel_timing).
void pf_kernel_mark(int kind, hipStream_t st, int end);
