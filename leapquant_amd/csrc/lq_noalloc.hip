// lq_decode_noalloc: one decode call (step, then the flush of the heads it made due) that allocates nothing and needs
// no workspace from the caller: the due list lives in this file's static device array.  For callers that cannot
// allocate device memory (code under graph capture, serving loops, harnesses that forbid hipMalloc).
#include "lq_common.h"

#include <mutex>

// {count of due heads, flush workgroups done, due list of p = n HV + hv}: zero at load, emptied again by every flush.
// One copy per GPU (256 KiB), held until the process ends and shared by every call on that GPU.  In host code the name
// stands for no device address: kernels and copies take the address hipGetSymbolAddress returns.
static __device__ __align__(256) int scratch[2 + LQ_DUE_MAX];

namespace {

constexpr int MAX_DEVICES = 64;

// Device address of this GPU's copy of `scratch`, looked up on the first call on the device (with it current).
int* scratch_on_current_device(int* status) {
  static std::mutex mu;
  static int* addr[MAX_DEVICES] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
    *status = LQ_ERR_HIP;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
      *status = LQ_ERR_HIP;
      return nullptr;
    }
    addr[dev] = (int*)p;
  }
  return addr[dev];
}

}  // namespace

extern "C" int lq_decode_noalloc(const lq_state* st, const lq_step_io* io, const float* Q0, int kda, float glb,
                                 void* stream) {
  int rc = lq_check_step(st, io);
  if (rc) return rc;
  if (kda != 0 && kda != 1) return LQ_ERR_ARG;
  if (kda && (!st->Gbuf || st->K != 128 || st->V != 128 || st->R > 4)) return LQ_ERR_ARG;
  const float qmax = st->qmax > 0.f ? st->qmax : LQ_QMAX;
  rc = lq_check_flush(st, Q0, io->idx, io->N, kda, qmax);
  if (rc) return rc;
  if ((long long)io->N * st->HV > LQ_DUE_MAX) return LQ_ERR_SIZE;   // more heads than the static due list holds
  // the list's address first, also for N = 0: a call with no rows, made before a graph capture, sets the device up
  // so that the captured calls make no runtime query
  int status = LQ_OK;
  int* dlist = scratch_on_current_device(&status);
  if (!dlist) return status;
  if (io->N == 0) return LQ_OK;
  hipStream_t s = (hipStream_t)stream;
  rc = lq_launch_step(st, io, kda, glb, dlist, s);
  if (rc) return rc;
  return lq_launch_flush(st, Q0, io->idx, io->N, kda, qmax, dlist, s);
}
