// resident.hip — host side of the resident decode loop (device code in
// resident.hpp, one kernel instantiation per row count in resident_k<MR>.hip).
#include <algorithm>

#include "resident.hpp"

namespace mitok {

// kernels of resident_k1/2/4/8.hip for a head dim (64 specialised, others
// generic), with the barrier or the polling exchange
const void* resident_kernel_1(int dh, bool poll);
const void* resident_kernel_2(int dh, bool poll);
const void* resident_kernel_4(int dh, bool poll);
const void* resident_kernel_8(int dh, bool poll);

static const void* pick_kernel(int mr, int dh, bool poll) {
  switch (mr) {
    case 1: return resident_kernel_1(dh, poll);
    case 2: return resident_kernel_2(dh, poll);
    case 4: return resident_kernel_4(dh, poll);
    default: return resident_kernel_8(dh, poll);
  }
}

bool resident_poll_built(int mr) { return pick_kernel(mr, 0, true) != nullptr; }

ResGemvPlan resident_gemv_plan(int M, int N, int K, bool part, int grid) {
  ResGemvPlan p;
  p.mr = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  p.C = 64;
  for (int c : {8, 16, 32, 64})
    if (rcdiv(N, c) <= grid) {
      p.C = c;
      break;
    }
  p.ncb = rcdiv(N, p.C);
  const int rpw = 64 / p.C;
  const int P = part ? std::min(8, std::max(1, grid / p.ncb)) : 1;
  if (p.ncb * P <= grid) {  // one item per block: the prefetched layout if it fits the registers
    const int kw3 = rcdiv(rcdiv(K, P), 3 * rpw) * rpw;
    if (kw3 / rpw <= RES_NPF) {
      p.waves = 3;
      p.kw = kw3;
      p.P = rcdiv(K, 3 * kw3);
      return p;
    }
  }
  p.waves = 4;
  const int unit = 4 * rpw;
  p.kw = rcdiv(rcdiv(K, P), unit) * unit / 4;
  p.P = rcdiv(K, 4 * p.kw);
  return p;
}

size_t resident_op_lds(const ROp& op) {
  const size_t att = op.ro.att.po ? (size_t)op.M * op.ro.att.H * (op.ro.att.nsplit + 1) * sizeof(double) : 0;
  if (op.kind == ROP_GEMV) {
    const int mr = op.M <= 1 ? 1 : op.M <= 2 ? 2 : op.M <= 4 ? 4 : 8;
    const size_t rl = op.ro.ln ? (size_t)op.K : (size_t)op.waves * op.kw;
    return (size_t)mr * rl * sizeof(double2) + att;
  }
  if (op.kind == ROP_ROWS) {
    const size_t rl = op.ro.ln ? (size_t)op.K : (size_t)std::min(op.cw, op.K);
    const size_t a1 = op.ro.att.po ? (size_t)op.ro.att.H * (op.ro.att.nsplit + 1) * sizeof(double) : 0;
    return rl * sizeof(double2) + a1;
  }
  return 0;
}

int resident_grid(int cus, bool cooperative, int mr, int dh, size_t shm, int* grid, bool poll) {
  if (!cooperative) return ERR_STATE;
  const void* k = pick_kernel(mr, dh, poll);
  if (!k) return ERR_STATE;
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k, 256, shm) != hipSuccess) {
    (void)hipGetLastError();  // a size the device refuses: no fault to report later
    return ERR_STATE;
  }
  if (occ < 1) return ERR_STATE;
  *grid = cus;
  return OK;
}

int resident_launch(hipStream_t st, const ROp* ops_d, int nops, int nsteps, const RStep& step, int mr, int dh,
                    size_t shm, int grid, uint32_t* flags, uint32_t epoch0, uint32_t* err, uint64_t* stamps,
                    bool poll) {
  if (nops <= 0 || nsteps <= 0) return OK;
  if (step.B < 1 || step.B > 8 || step.B > mr) return ERR_ARG;
  if (poll && (!step.arena || step.arena_half <= 0 || !step.part_v1 || !step.part_i1)) return ERR_ARG;
  const void* k = pick_kernel(mr, dh, poll);
  if (!k) return ERR_STATE;
  RStep sa = step;
  void* args[] = {(void*)&ops_d, (void*)&nops, (void*)&nsteps, (void*)&sa, (void*)&flags, (void*)&epoch0, (void*)&err,
                  (void*)&stamps};
  if (hipLaunchCooperativeKernel(k, dim3(grid), dim3(256), args, (unsigned)shm, st) != hipSuccess) return ERR_HIP;
  return OK;
}

// rows [kv_len[b], kv_len[b] + n) of every (sequence, head) cache, clipped to
// ctx, set to the sentinel; one thread per complex element
__global__ __launch_bounds__(256) void k_kv_sentinel(double2* kc, double2* vc, int H, int ctx, int dh,
                                                     const int* kv_len, int n, long total) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const long per_seq = (long)H * n * dh;
  const int b = (int)(i / per_seq);
  const long r = i - b * per_seq;
  const int h = (int)(r / ((long)n * dh));
  const long r2 = r - (long)h * n * dh;
  const int j = (int)(r2 / dh), e = (int)(r2 - (long)j * dh);
  const int p = kv_len[b] + j;
  if (p < 0 || p >= ctx) return;
  const long at = (((long)b * H + h) * ctx + p) * dh + e;
  const double s = __longlong_as_double((long long)RES_SENT);
  kc[at] = make_double2(s, s);
  vc[at] = make_double2(s, s);
}

void resident_kv_sentinel(hipStream_t st, double2* kc, double2* vc, int B, int H, int ctx, int dh, const int* kv_len,
                          int n) {
  const long total = (long)B * H * n * dh;
  if (total <= 0) return;
  MITOK_LAUNCH(k_kv_sentinel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, kc, vc, H, ctx, dh, kv_len, n,
               total);
}

}  // namespace mitok
