// Value statistics of the layer's input tensors in one pass: for each of up
// to kMaxStatTensors contiguous float32 / float64 tensors, (min, max,
// non-finite count > 0).  bayesian_layer's argument checks (finite entries,
// variance signs; bayes_ssm/bayesian_layer.py:105-129, :798-985) read them
// back with one device->host copy instead of one reduction launch and one
// synchronization per tensor.
//
// Pass 1: every block takes kChunk consecutive elements of one tensor (16-byte
// loads where the tensor allows it), reduces its threads' (min, max, bad) in
// LDS and writes one partial.  Pass 2: one block per tensor folds its
// partials.  min and max skip NaN and infinities, which set `bad` instead, so
// the host sees every failing case.

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "bssm_recurrence.h"

namespace bssm {
namespace checks {
namespace {

constexpr int kThreads = 256;
constexpr int64_t kChunk = 16384;  // elements per pass-1 block

struct Acc {
  float lo, hi, bad;
  __device__ __forceinline__ void add(float x) {
    // x - x is 0 for finite x and NaN otherwise.
    if ((x - x) != 0.f) {
      bad = 1.f;
    } else {
      lo = fminf(lo, x);
      hi = fmaxf(hi, x);
    }
  }
  // float64 entries are folded as float32 values with their sign: clamped to
  // the float32 range, and a nonzero value that rounds to zero kept at
  // +-FLT_MIN.  The host tests only finiteness (decided here, on the double)
  // and signs, which this mapping preserves.
  __device__ __forceinline__ void add(double x) {
    if ((x - x) != 0.0) {
      bad = 1.f;
    } else {
      float f = static_cast<float>(fmin(fmax(x, -static_cast<double>(FLT_MAX)), static_cast<double>(FLT_MAX)));
      if (f == 0.f && x != 0.0) f = x > 0.0 ? FLT_MIN : -FLT_MIN;
      lo = fminf(lo, f);
      hi = fmaxf(hi, f);
    }
  }
  __device__ __forceinline__ void merge(const Acc& o) {
    lo = fminf(lo, o.lo);
    hi = fmaxf(hi, o.hi);
    bad = fmaxf(bad, o.bad);
  }
};

__device__ __forceinline__ Acc block_reduce(Acc a, float* red) {
  const int t = threadIdx.x;
  red[t] = a.lo;
  red[kThreads + t] = a.hi;
  red[2 * kThreads + t] = a.bad;
  __syncthreads();
  for (int w = kThreads / 2; w > 0; w >>= 1) {
    if (t < w) {
      red[t] = fminf(red[t], red[t + w]);
      red[kThreads + t] = fmaxf(red[kThreads + t], red[kThreads + t + w]);
      red[2 * kThreads + t] = fmaxf(red[2 * kThreads + t], red[2 * kThreads + t + w]);
    }
    __syncthreads();
  }
  return Acc{red[0], red[kThreads], red[2 * kThreads]};
}

__global__ __launch_bounds__(kThreads) void partial_kernel(StatArgs a, float* __restrict__ part) {
  __shared__ float red[3 * kThreads];
  const int64_t blk = blockIdx.x;
  int ti = 0;
  while (ti + 1 < a.count && blk >= a.first_block[ti + 1]) ++ti;
  const int64_t start = (blk - a.first_block[ti]) * kChunk;
  const int64_t n = a.numel[ti];
  const int64_t end = start + kChunk < n ? start + kChunk : n;
  Acc acc{FLT_MAX, -FLT_MAX, 0.f};
  if (a.is_double[ti]) {
    const double* x = static_cast<const double*>(a.ptr[ti]);
    for (int64_t i = start + threadIdx.x; i < end; i += kThreads) acc.add(x[i]);
  } else {
    const float* x = static_cast<const float*>(a.ptr[ti]);
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    int64_t i = start + 4 * threadIdx.x;
    if (vec) {
      typedef float v4 __attribute__((ext_vector_type(4)));
      for (; i + 3 < end; i += 4 * kThreads) {
        const v4 v = __builtin_nontemporal_load(reinterpret_cast<const v4*>(x + i));
        acc.add(v[0]);
        acc.add(v[1]);
        acc.add(v[2]);
        acc.add(v[3]);
      }
      // The tail of the tensor (fewer than 4 elements) after the last whole piece.
      const int64_t tail = end - (end - start) % 4;
      for (int64_t k = tail + threadIdx.x; k < end; k += kThreads) acc.add(x[k]);
    } else {
      for (int64_t k = start + threadIdx.x; k < end; k += kThreads) acc.add(x[k]);
    }
  }
  const Acc r = block_reduce(acc, red);
  if (threadIdx.x == 0) {
    part[3 * blk] = r.lo;
    part[3 * blk + 1] = r.hi;
    part[3 * blk + 2] = r.bad;
  }
}

__global__ __launch_bounds__(kThreads) void fold_kernel(StatArgs a, const float* __restrict__ part,
                                                        float* __restrict__ out) {
  __shared__ float red[3 * kThreads];
  const int ti = blockIdx.x;
  const int64_t b0 = a.first_block[ti];
  const int64_t b1 = ti + 1 < a.count ? a.first_block[ti + 1] : a.total_blocks;
  Acc acc{FLT_MAX, -FLT_MAX, 0.f};
  for (int64_t b = b0 + threadIdx.x; b < b1; b += kThreads)
    acc.merge(Acc{part[3 * b], part[3 * b + 1], part[3 * b + 2]});
  const Acc r = block_reduce(acc, red);
  if (threadIdx.x == 0) {
    out[3 * ti] = r.lo;
    out[3 * ti + 1] = r.hi;
    out[3 * ti + 2] = r.bad;
  }
}

}  // namespace
}  // namespace checks

int64_t stat_blocks(int64_t numel) { return (numel + checks::kChunk - 1) / checks::kChunk; }

hipError_t launch_value_stats(const StatArgs& a, float* partials, float* out, hipStream_t stream) {
  if (a.count == 0) return hipSuccess;
  if (a.total_blocks > 0) {
    hipLaunchKernelGGL(checks::partial_kernel, dim3(static_cast<unsigned>(a.total_blocks)), dim3(checks::kThreads),
                       0, stream, a, partials);
  }
  hipLaunchKernelGGL(checks::fold_kernel, dim3(static_cast<unsigned>(a.count)), dim3(checks::kThreads), 0, stream, a,
                     partials, out);
  return hipGetLastError();
}

}  // namespace bssm
