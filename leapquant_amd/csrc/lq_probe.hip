// Streaming-read probe: what this GPU's memory system delivers for a given read pattern, the ceiling against which the
// decode step's achieved bandwidth is read.  Measurement only (bench.py); not part of liblq's API.
//
// Every workgroup (256 threads) reads bytes [0, nbytes) of `per_wg` consecutive blocks, block b at base + b * stride,
// with 16-byte loads, eight in flight per thread (plain or with the non-temporal hint), and folds them into one word
// that is stored only if it equals a constant no data produces in practice, so nothing is written and no load is dead.
// nblocks = 0 launches one empty workgroup: the fixed cost of a launch.  lq_probe_rmw reads the same way and writes
// every 16 bytes back in place XOR `key` (0: the data is unchanged): the read-modify-write stream of a dense-state step.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__global__ __launch_bounds__(256) void probe_read_kernel(const char* __restrict__ base, long long stride, int nbytes,
                                                         int nblocks, int per_wg, unsigned* __restrict__ sink) {
  const int n16 = nbytes >> 4;
  unsigned acc = 0;
  for (int k = 0; k < per_wg; ++k) {
    const int b = blockIdx.x * per_wg + k;
    if (b >= nblocks) break;
    const u32x4* p = (const u32x4*)(base + (long long)b * stride);
    for (int i0 = threadIdx.x; i0 < n16; i0 += 8 * 256) {
      u32x4 x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = min(i0 + 256 * u, n16 - 1);            // clamped: in bounds, the surplus re-reads the last chunk
        x[u] = NT ? __builtin_nontemporal_load(p + i) : p[i];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) acc ^= x[u].x ^ x[u].y ^ x[u].z ^ x[u].w;
    }
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x * 256 + threadIdx.x] = acc;
}

template <bool NT>
__global__ __launch_bounds__(256) void probe_rmw_kernel(char* __restrict__ base, long long stride, int nbytes,
                                                        int nblocks, int per_wg, unsigned key) {
  const int n16 = nbytes >> 4;
  for (int k = 0; k < per_wg; ++k) {
    const int b = blockIdx.x * per_wg + k;
    if (b >= nblocks) break;
    u32x4* p = (u32x4*)(base + (long long)b * stride);
    for (int i0 = threadIdx.x; i0 < n16; i0 += 8 * 256) {
      u32x4 x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = min(i0 + 256 * u, n16 - 1);
        x[u] = NT ? __builtin_nontemporal_load(p + i) : p[i];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = i0 + 256 * u;
        if (i < n16) {
          const u32x4 y = x[u] ^ key;
          if (NT) __builtin_nontemporal_store(y, p + i);
          else p[i] = y;
        }
      }
    }
  }
}

}  // namespace

// 0 ok, -1 bad argument, -2 launch error.  sink: at least ceil(nblocks / per_wg) * 256 words (never written in practice).
extern "C" int lq_probe_read(const void* base, long long stride, int nbytes, int nblocks, int per_wg, int nontemporal,
                             unsigned* sink, void* stream) {
  if (nblocks < 0 || per_wg < 1 || nbytes < 16 || (nbytes & 15) || stride < nbytes || (stride & 15)) return -1;
  if (nblocks > 0 && (!base || !sink || ((uintptr_t)base & 15))) return -1;
  const unsigned grid = nblocks > 0 ? (unsigned)((nblocks + per_wg - 1) / per_wg) : 1u;
  hipStream_t s = (hipStream_t)stream;
  if (nontemporal) probe_read_kernel<true><<<grid, 256, 0, s>>>((const char*)base, stride, nbytes, nblocks, per_wg, sink);
  else probe_read_kernel<false><<<grid, 256, 0, s>>>((const char*)base, stride, nbytes, nblocks, per_wg, sink);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// the read-modify-write stream: 0 ok, -1 bad argument, -2 launch error
extern "C" int lq_probe_rmw(void* base, long long stride, int nbytes, int nblocks, int per_wg, int nontemporal,
                            unsigned key, void* stream) {
  if (nblocks < 1 || per_wg < 1 || nbytes < 16 || (nbytes & 15) || stride < nbytes || (stride & 15) || !base ||
      ((uintptr_t)base & 15))
    return -1;
  const unsigned grid = (unsigned)((nblocks + per_wg - 1) / per_wg);
  hipStream_t s = (hipStream_t)stream;
  if (nontemporal) probe_rmw_kernel<true><<<grid, 256, 0, s>>>((char*)base, stride, nbytes, nblocks, per_wg, key);
  else probe_rmw_kernel<false><<<grid, 256, 0, s>>>((char*)base, stride, nbytes, nblocks, per_wg, key);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}
