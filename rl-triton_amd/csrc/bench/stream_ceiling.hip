// stream_ceiling.hip -- the streaming ceiling of a return-estimation kernel's byte
// pattern: n_in reads and n_out writes of float32 arrays, one 16-byte non-temporal access
// per array per thread, 512-thread workgroups, no scan.  The benchmark times it on the
// same rotating HBM-resident inputs as the scan kernels and reports each kernel's time
// against it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rlk_stream_ceiling.h"

namespace {

constexpr int kThreads = 512;
typedef float f4 __attribute__((ext_vector_type(4)));

struct Ptrs {
  const f4* in[6];
  f4* out[2];
};

// The loads are unconditional (a thread past the end reads the last vector) and only the
// stores are guarded: with an early return first, the compiler loaded the array pointers
// only after the bounds check, so every wave waited on two scalar loads of the kernel
// arguments in a row before its first load (0.33 us per launch at the V-trace pattern's
// headline size).
template <int NR, int NW>
__global__ __launch_bounds__(kThreads) void stream_kernel(Ptrs p, int64_t n4) {
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t i = i0 < n4 ? i0 : n4 - 1;
  f4 v[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) v[k] = __builtin_nontemporal_load(p.in[k] + i);
  f4 s = v[0];
#pragma unroll
  for (int k = 1; k < NR; ++k) s += v[k];
  asm volatile("" ::: "memory");  // keeps the loads (and their pointers) ahead of the check
  if (i0 >= n4) return;
#pragma unroll
  for (int k = 0; k < NW; ++k) __builtin_nontemporal_store(s * static_cast<float>(k + 1), p.out[k] + i);
}

template <int NR, int NW>
int launch(const Ptrs& p, int64_t n4, hipStream_t s) {
  const int64_t blocks = (n4 + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) return -1;
  hipLaunchKernelGGL((stream_kernel<NR, NW>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s, p, n4);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

template <int NW>
int by_reads(int n_in, const Ptrs& p, int64_t n4, hipStream_t s) {
  switch (n_in) {
    case 1: return launch<1, NW>(p, n4, s);
    case 2: return launch<2, NW>(p, n4, s);
    case 3: return launch<3, NW>(p, n4, s);
    case 4: return launch<4, NW>(p, n4, s);
    case 5: return launch<5, NW>(p, n4, s);
    case 6: return launch<6, NW>(p, n4, s);
  }
  return -1;
}

bool aligned(const void* q) { return q != nullptr && (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

}  // namespace

extern "C" int rlk_stream_ceiling(const float* const* in, int n_in, float* const* out, int n_out,
                                  int64_t n, void* stream) {
  if (in == nullptr || out == nullptr || n_in < 1 || n_in > 6 || n_out < 1 || n_out > 2 || n < 0 ||
      n % 4 != 0)
    return -1;
  Ptrs p{};
  for (int k = 0; k < n_in; ++k) {
    if (!aligned(in[k])) return -1;
    p.in[k] = reinterpret_cast<const f4*>(in[k]);
  }
  for (int k = 0; k < n_out; ++k) {
    if (!aligned(out[k])) return -1;
    p.out[k] = reinterpret_cast<f4*>(out[k]);
  }
  if (n == 0) return 0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return n_out == 1 ? by_reads<1>(n_in, p, n / 4, s) : by_reads<2>(n_in, p, n / 4, s);
}
