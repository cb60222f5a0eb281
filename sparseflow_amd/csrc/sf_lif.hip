// Standalone multi-step LIF neuron: x [T, m] input currents -> spikes [T, m]
// and the membrane after step T.  The neuron layers of a spiking network
// between (and after) the sparse convolutions; spikingjelly's multi-step
// LIFNode in the reference's models (Benchmark/bench_4test.py:166-197,
// Core/registry.py:22-29), with the update rule the reference restates in
// Ops/sparse_fused_conv_lif.py:283-292.
//
// One thread owns VEC consecutive neurons for all T steps; the membrane stays
// in registers, x_t+1 is loaded while step t is computed, x and the spikes
// are streamed once (non-temporal).  HBM-bound: T*m*(|x| + |spike|) + 4m
// (+ 4m for v_init) bytes.
//
// The arithmetic is the LIFNode torch path's, operation by operation, with
// no fused multiply-adds (the torch path rounds after every tensor op), so
// both give bit-identical spikes and membranes.
#include <algorithm>

#include "sf_internal.h"

namespace sf {

namespace {

template <typename T, int VEC>
struct Vec;
template <>
struct Vec<float, 4> {
  typedef float type __attribute__((ext_vector_type(4)));
};

template <typename TIn, int VEC>
__device__ __forceinline__ void lif_load(const TIn* __restrict__ p, float (&v)[VEC]) {
  if constexpr (VEC == 4 && sizeof(TIn) == 4) {
    typedef typename Vec<float, 4>::type f4;
    const f4 q = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) v[i] = to_f32<TIn>(p[i]);
  }
}

template <typename TOut, int VEC>
__device__ __forceinline__ void lif_store(TOut* __restrict__ p, const float (&s)[VEC]) {
  if constexpr (VEC == 4 && sizeof(TOut) == 4) {
    typedef typename Vec<float, 4>::type f4;
    f4 q;
    q.x = s[0]; q.y = s[1]; q.z = s[2]; q.w = s[3];
    __builtin_nontemporal_store(q, reinterpret_cast<f4*>(p));
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) p[i] = from_f32<TOut>(s[i]);
  }
}

struct LifRun {
  int64_t m;
  int T;
  float tau, v_th, v_reset, vr, v0;
  int hard, decay_input;
};

#pragma clang fp contract(off)
__device__ __forceinline__ float lif_charge(const LifRun& r, float v, float x) {
  return r.decay_input ? v + (x - (v - r.vr)) / r.tau : v - (v - r.vr) / r.tau + x;
}

template <typename TIn, typename TOut, int VEC>
__global__ __launch_bounds__(256) void k_lif_multistep(const TIn* __restrict__ x, const float* __restrict__ v_init,
                                                       TOut* __restrict__ spikes, float* __restrict__ v_out,
                                                       LifRun r) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * VEC;
  for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * VEC; i < r.m; i += stride) {
    float v[VEC], xn[VEC];
    if (v_init != nullptr) {
#pragma unroll
      for (int k = 0; k < VEC; ++k) v[k] = v_init[i + k];
    } else {
#pragma unroll
      for (int k = 0; k < VEC; ++k) v[k] = r.v0;
    }
    lif_load<TIn, VEC>(x + i, xn);
    for (int t = 0; t < r.T; ++t) {
      float xc[VEC];
#pragma unroll
      for (int k = 0; k < VEC; ++k) xc[k] = xn[k];
      if (t + 1 < r.T) lif_load<TIn, VEC>(x + (int64_t)(t + 1) * r.m + i, xn);
      float s[VEC];
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        const float h = lif_charge(r, v[k], xc[k]);
        const bool fire = h >= r.v_th;
        s[k] = fire ? 1.f : 0.f;
        v[k] = r.hard ? (fire ? r.v_reset : h) : h - s[k] * r.v_th;
      }
      lif_store<TOut, VEC>(spikes + (int64_t)t * r.m + i, s);
    }
#pragma unroll
    for (int k = 0; k < VEC; ++k) v_out[i + k] = v[k];
  }
}

template <typename TIn, typename TOut>
int launch_lif_ms_t(const void* x, const float* v_init, void* spikes, float* v_out, const LifRun& r,
                    hipStream_t stream) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(spikes) |
                       reinterpret_cast<uintptr_t>(v_out) | reinterpret_cast<uintptr_t>(v_init);
  const bool vec4 = r.m % 4 == 0 && (al % 16) == 0;
  const int vec = vec4 ? 4 : 1;
  const int64_t threads = (r.m + vec - 1) / vec;
  // Enough blocks to fill the chip several times; the loop strides the rest.
  const int64_t max_blocks = 256LL * 32;
  const int64_t blocks = std::min<int64_t>((threads + 255) / 256, max_blocks);
  if (blocks == 0) return (int)hipSuccess;
  if (vec4)
    hipLaunchKernelGGL((k_lif_multistep<TIn, TOut, 4>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const TIn*>(x), v_init, static_cast<TOut*>(spikes), v_out, r);
  else
    hipLaunchKernelGGL((k_lif_multistep<TIn, TOut, 1>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const TIn*>(x), v_init, static_cast<TOut*>(spikes), v_out, r);
  return (int)hipGetLastError();
}

}  // namespace

int launch_lif_multistep(const void* x, int in_dtype, int T, int64_t m, float tau, float v_th, float v_reset,
                         int hard_reset, int decay_input, const float* v_init, void* spikes, int out_dtype,
                         float* v_out, hipStream_t stream) {
  LifRun r;
  r.m = m;
  r.T = T;
  r.tau = tau;
  r.v_th = v_th;
  r.v_reset = v_reset;
  r.hard = hard_reset != 0;
  r.decay_input = decay_input != 0;
  r.vr = r.hard ? v_reset : 0.f;
  r.v0 = r.hard ? v_reset : 0.f;
  timing_begin(K_LIF_MS, stream);
  int rc;
  if (in_dtype == SF_F16)
    rc = out_dtype == SF_F32 ? launch_lif_ms_t<__half, float>(x, v_init, spikes, v_out, r, stream)
                             : launch_lif_ms_t<__half, __half>(x, v_init, spikes, v_out, r, stream);
  else if (in_dtype == SF_BF16)
    rc = out_dtype == SF_F32 ? launch_lif_ms_t<__hip_bfloat16, float>(x, v_init, spikes, v_out, r, stream)
                             : launch_lif_ms_t<__hip_bfloat16, __hip_bfloat16>(x, v_init, spikes, v_out, r, stream);
  else
    rc = launch_lif_ms_t<float, float>(x, v_init, spikes, v_out, r, stream);
  timing_end(K_LIF_MS, stream);
  return rc;
}

}  // namespace sf
