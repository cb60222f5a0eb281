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
// (+ 4m for v_init) bytes.  Optional extras: a second input summed into the
// current (the residual add before a block's last neuron layer, fused) and
// the spike map of the output in the prescan's bitmap layout.
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

// Input current of step t (x, plus x2 when given: the residual sum x + x2
// rounded once, as the torch expression `out + identity` does).
template <typename TIn, int VEC>
__device__ __forceinline__ void lif_input(const TIn* __restrict__ x, const TIn* __restrict__ x2, int64_t off,
                                          float (&v)[VEC]) {
  lif_load<TIn, VEC>(x + off, v);
  if (x2 != nullptr) {
    float w[VEC];
    lif_load<TIn, VEC>(x2 + off, w);
#pragma unroll
    for (int k = 0; k < VEC; ++k) v[k] = to_f32<TIn>(from_f32<TIn>(v[k] + w[k]));
  }
}

template <typename TIn, typename TOut, int VEC>
__global__ __launch_bounds__(256) void k_lif_multistep(const TIn* __restrict__ x, const TIn* __restrict__ x2,
                                                       const float* __restrict__ v_init,
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
    lif_input<TIn, VEC>(x, x2, i, xn);
    for (int t = 0; t < r.T; ++t) {
      float xc[VEC];
#pragma unroll
      for (int k = 0; k < VEC; ++k) xc[k] = xn[k];
      if (t + 1 < r.T) lif_input<TIn, VEC>(x, x2, (int64_t)(t + 1) * r.m + i, xn);
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

// The same neuron update laid out as the prescan: thread = (sample n,
// bitmap word w, pixel p) owns 32 channels of one pixel for all T steps and
// also writes the spike map word of each step (bit c & 31 of word c >> 5 of
// pixel p of frame t*N + n), so the next sparse convolution can skip its
// prescan.  Consecutive threads take consecutive pixels: every channel
// plane is read and written in 256-byte runs.  Word w of pixel p of a frame
// sits at p * ps + w * ws words from the frame's start: (cwp, 1) pixel-major,
// (1, hw) as word planes.
struct LifMap {
  int64_t n, hw;
  int c, cwp;
  int64_t ps, ws;
};

template <typename TIn, typename TOut>
__global__ __launch_bounds__(256) void k_lif_bits(const TIn* __restrict__ x, const TIn* __restrict__ x2,
                                                  const float* __restrict__ v_init, TOut* __restrict__ spikes,
                                                  float* __restrict__ v_out, uint32_t* __restrict__ bits,
                                                  uint32_t* __restrict__ flags, int64_t nflags, LifRun r, LifMap g) {
  // Every chunk of a spike map is binary.
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nflags; i += (int64_t)gridDim.x * blockDim.x)
    flags[i] = 0u;
  // Wave tile = 64 consecutive pixels of one (sample, word): sample, word
  // and channel bases are wave-uniform (scalar), the lane adds its pixel.
  const int lane = lane_id();
  const int64_t tiles_per_word = (g.hw + 63) / 64;
  const int64_t ntiles = g.n * g.cwp * tiles_per_word;
  const int64_t wave0 = (int64_t)blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t wstride = (int64_t)gridDim.x * (blockDim.x >> 6);
  for (int64_t wt = wave0; wt < ntiles; wt += wstride) {
    const int64_t nw = wt / tiles_per_word;
    const int64_t p = (wt - nw * tiles_per_word) * 64 + lane;
    const int w = (int)(nw % g.cwp);
    const int64_t n = nw / g.cwp;
    const int c0 = w * 32;
    const int nc = max(0, min(32, g.c - c0));  // channels in this word (0 for padding words)
    const bool px = p < g.hw;
    const uint32_t pl = px ? (uint32_t)p : 0u;  // pixel read (last lanes of a ragged tile re-read pixel 0)
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = r.v0;
    if (v_init != nullptr && px) {
#pragma unroll
      for (int j = 0; j < 32; ++j)
        if (j < nc) v[j] = v_init[(n * g.c + c0 + j) * g.hw + p];
    }
    // Step t+1's currents are loaded before step t's spikes are stored (the
    // memory counter is in order: a wait for loads issued after the stores
    // would also wait for the stores).  Padding channels re-read channel c0
    // and are discarded.
    float xa[32], xb[32];
    auto load_step = [&](int t) {
      const TIn* xr = x + (((int64_t)t * g.n + n) * g.c + c0) * g.hw;
      const TIn* xr2 = x2 + (((int64_t)t * g.n + n) * g.c + c0) * g.hw;
      // Scalar channel-plane base + 32-bit lane offset per load.
#pragma unroll
      for (int j = 0; j < 32; ++j) xa[j] = to_f32<TIn>((xr + (int64_t)(j < nc ? j : 0) * g.hw)[pl]);
      if (x2 != nullptr) {
#pragma unroll
        for (int j = 0; j < 32; ++j) xb[j] = to_f32<TIn>((xr2 + (int64_t)(j < nc ? j : 0) * g.hw)[pl]);
      }
    };
    load_step(0);
    for (int t = 0; t < r.T; ++t) {
      float xc[32];
#pragma unroll
      for (int j = 0; j < 32; ++j) xc[j] = x2 != nullptr ? to_f32<TIn>(from_f32<TIn>(xa[j] + xb[j])) : xa[j];
      if (t + 1 < r.T) load_step(t + 1);
      const int64_t f = (int64_t)t * g.n + n;
      TOut* sr = spikes + (f * g.c + c0) * g.hw;
      uint32_t word = 0u;
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        const float h = lif_charge(r, v[j], xc[j]);
        const bool fire = h >= r.v_th;
        const float sp = fire ? 1.f : 0.f;
        v[j] = r.hard ? (fire ? r.v_reset : h) : h - sp * r.v_th;
        if (j < nc && px) (sr + (int64_t)j * g.hw)[pl] = from_f32<TOut>(sp);
        word |= (fire && j < nc ? 1u : 0u) << j;
      }
      if (px) bits[f * g.hw * g.cwp + p * g.ps + w * g.ws] = word;
    }
    if (px) {
#pragma unroll
      for (int j = 0; j < 32; ++j)
        if (j < nc) v_out[(n * g.c + c0 + j) * g.hw + p] = v[j];
    }
  }
}

// Vector form for planes with h*w % 4 == 0: a block of 4 wavefronts owns 256
// consecutive pixels of one (sample, word) -- each wavefront 8 of the word's
// 32 channels, each lane 4 pixels (16-byte loads and stores) -- and the
// four partial words of a pixel are OR-ed in LDS once per step.
template <typename TIn, typename TOut>
__global__ __launch_bounds__(256) void k_lif_bits4(const TIn* __restrict__ x, const TIn* __restrict__ x2,
                                                   const float* __restrict__ v_init, TOut* __restrict__ spikes,
                                                   float* __restrict__ v_out, uint32_t* __restrict__ bits,
                                                   uint32_t* __restrict__ flags, int64_t nflags, LifRun r, LifMap g) {
  __shared__ uint32_t s_word[256];
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nflags; i += (int64_t)gridDim.x * blockDim.x)
    flags[i] = 0u;
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t tiles_per_word = (g.hw + 255) / 256;
  const int64_t ntiles = g.n * g.cwp * tiles_per_word;
  for (int64_t bt = blockIdx.x; bt < ntiles; bt += gridDim.x) {
    const int64_t nw = bt / tiles_per_word;
    const int64_t p0 = (bt - nw * tiles_per_word) * 256;
    const int w = (int)(nw % g.cwp);
    const int64_t n = nw / g.cwp;
    const int cw0 = w * 32 + wave * 8;                     // this wavefront's first channel
    const int nc = max(0, min(8, g.c - cw0));              // its channels (0 past C)
    const int64_t p = p0 + 4 * lane;
    const bool px = p < g.hw;                              // hw % 4 == 0: all 4 pixels or none
    const int64_t pl = px ? p : 0;
    float v[8][4];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[j][e] = r.v0;
    if (v_init != nullptr && px) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < nc) {
          float q[4];
          lif_load<float, 4>(v_init + (n * g.c + cw0 + j) * g.hw + p, q);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[j][e] = q[e];
        }
    }
    float xa[8][4], xb[8][4];
    auto load_step = [&](int t) {
      const int64_t base = (((int64_t)t * g.n + n) * g.c) * g.hw + pl;
#pragma unroll
      for (int j = 0; j < 8; ++j) lif_load<TIn, 4>(x + base + (int64_t)(cw0 + (j < nc ? j : 0)) * g.hw, xa[j]);
      if (x2 != nullptr) {
#pragma unroll
        for (int j = 0; j < 8; ++j) lif_load<TIn, 4>(x2 + base + (int64_t)(cw0 + (j < nc ? j : 0)) * g.hw, xb[j]);
      }
    };
    if (nc > 0) load_step(0);
    for (int t = 0; t < r.T; ++t) {
      const int64_t f = (int64_t)t * g.n + n;
      s_word[threadIdx.x] = 0u;
      __syncthreads();
      uint32_t part[4] = {0u, 0u, 0u, 0u};
      if (nc > 0) {
        float xc[8][4];
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            xc[j][e] = x2 != nullptr ? to_f32<TIn>(from_f32<TIn>(xa[j][e] + xb[j][e])) : xa[j][e];
        if (t + 1 < r.T) load_step(t + 1);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float sp[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float h = lif_charge(r, v[j][e], xc[j][e]);
            const bool fire = h >= r.v_th;
            sp[e] = fire ? 1.f : 0.f;
            v[j][e] = r.hard ? (fire ? r.v_reset : h) : h - sp[e] * r.v_th;
            part[e] |= (fire && j < nc ? 1u : 0u) << (wave * 8 + j);
          }
          if (j < nc && px) lif_store<TOut, 4>(spikes + (f * g.c + cw0 + j) * g.hw + p, sp);
        }
        if (px) {
#pragma unroll
          for (int e = 0; e < 4; ++e) atomicOr(&s_word[4 * lane + e], part[e]);
        }
      }
      __syncthreads();
      const int64_t pw = p0 + threadIdx.x;
      if (pw < g.hw) bits[f * g.hw * g.cwp + pw * g.ps + w * g.ws] = s_word[threadIdx.x];
      __syncthreads();
    }
    if (px) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < nc) {
          float* vo = v_out + (n * g.c + cw0 + j) * g.hw + p;
#pragma unroll
          for (int e = 0; e < 4; ++e) vo[e] = v[j][e];
        }
    }
  }
}

template <typename TIn, typename TOut>
int launch_lif_bits_t(const void* x, const void* x2, const float* v_init, void* spikes, float* v_out, uint32_t* bits,
                      uint32_t* flags, int64_t nflags, const LifRun& r, const LifMap& g, hipStream_t stream) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(x2) |
                       reinterpret_cast<uintptr_t>(spikes) | reinterpret_cast<uintptr_t>(v_out) |
                       reinterpret_cast<uintptr_t>(v_init);
  if (g.hw % 4 == 0 && (al % 16) == 0) {
    const int64_t tiles = g.n * g.cwp * ((g.hw + 255) / 256);
    const int64_t blocks = std::min<int64_t>(std::max<int64_t>(tiles, 1), 256LL * 64);
    hipLaunchKernelGGL((k_lif_bits4<TIn, TOut>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const TIn*>(x), static_cast<const TIn*>(x2), v_init, static_cast<TOut*>(spikes),
                       v_out, bits, flags, nflags, r, g);
    return (int)hipGetLastError();
  }
  const int64_t waves = g.n * g.cwp * ((g.hw + 63) / 64);
  const int64_t blocks = std::min<int64_t>(std::max<int64_t>((waves + 3) / 4, 1), 256LL * 32);
  hipLaunchKernelGGL((k_lif_bits<TIn, TOut>), dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const TIn*>(x), static_cast<const TIn*>(x2), v_init, static_cast<TOut*>(spikes),
                     v_out, bits, flags, nflags, r, g);
  return (int)hipGetLastError();
}

template <typename TIn, typename TOut>
int launch_lif_ms_t(const void* x, const void* x2, const float* v_init, void* spikes, float* v_out, const LifRun& r,
                    hipStream_t stream) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(x2) |
                       reinterpret_cast<uintptr_t>(spikes) | reinterpret_cast<uintptr_t>(v_out) |
                       reinterpret_cast<uintptr_t>(v_init);
  const bool vec4 = r.m % 4 == 0 && (al % 16) == 0;
  const int vec = vec4 ? 4 : 1;
  const int64_t threads = (r.m + vec - 1) / vec;
  // Enough blocks to fill the chip several times; the loop strides the rest.
  const int64_t max_blocks = 256LL * 32;
  const int64_t blocks = std::min<int64_t>((threads + 255) / 256, max_blocks);
  if (blocks == 0) return (int)hipSuccess;
  if (vec4)
    hipLaunchKernelGGL((k_lif_multistep<TIn, TOut, 4>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const TIn*>(x), static_cast<const TIn*>(x2), v_init, static_cast<TOut*>(spikes),
                       v_out, r);
  else
    hipLaunchKernelGGL((k_lif_multistep<TIn, TOut, 1>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const TIn*>(x), static_cast<const TIn*>(x2), v_init, static_cast<TOut*>(spikes),
                       v_out, r);
  return (int)hipGetLastError();
}

}  // namespace

int launch_lif_multistep(const void* x, const void* x2, int in_dtype, int T, int64_t n, int c, int64_t hw, float tau,
                         float v_th, float v_reset, int hard_reset, int decay_input, const float* v_init, void* spikes,
                         int out_dtype, float* v_out, uint32_t* bits, int cwp, int planes, uint32_t* flags,
                         int64_t nflags, hipStream_t stream) {
  LifRun r;
  r.m = n * c * hw;
  r.T = T;
  r.tau = tau;
  r.v_th = v_th;
  r.v_reset = v_reset;
  r.hard = hard_reset != 0;
  r.decay_input = decay_input != 0;
  r.vr = r.hard ? v_reset : 0.f;
  r.v0 = r.hard ? v_reset : 0.f;
  LifMap g;
  g.n = n;
  g.hw = hw;
  g.c = c;
  g.cwp = cwp;
  g.ps = planes ? 1 : cwp;
  g.ws = planes ? hw : 1;
#define SF_LIF_LAUNCH(TI, TO)                                                                   \
  (bits != nullptr ? launch_lif_bits_t<TI, TO>(x, x2, v_init, spikes, v_out, bits, flags, nflags, r, g, stream) \
                   : launch_lif_ms_t<TI, TO>(x, x2, v_init, spikes, v_out, r, stream))
  timing_begin(K_LIF_MS, stream);
  int rc;
  if (in_dtype == SF_F16)
    rc = out_dtype == SF_F32 ? SF_LIF_LAUNCH(__half, float) : SF_LIF_LAUNCH(__half, __half);
  else if (in_dtype == SF_BF16)
    rc = out_dtype == SF_F32 ? SF_LIF_LAUNCH(__hip_bfloat16, float) : SF_LIF_LAUNCH(__hip_bfloat16, __hip_bfloat16);
  else
    rc = SF_LIF_LAUNCH(float, float);
  timing_end(K_LIF_MS, stream);
#undef SF_LIF_LAUNCH
  return rc;
}

// ---------------------------------------------------------------------------
// Max pooling of a binary spike tensor given by its spike map (the pixel-major
// words a neuron layer hands over): the max of 0/1 values over a window is
// the OR of the window's words, so the pooled spikes and their own map come
// from the words alone (cwp words per input pixel read, no float input).
// One thread per output pixel: the OR of its window's in-frame words is
// written as the output map's words and, one channel plane per store
// (consecutive threads = consecutive pixels of the plane), as 0 / 1 values.
// ---------------------------------------------------------------------------
namespace {

template <typename TOut>
__global__ __launch_bounds__(256) void k_spike_maxpool(const uint32_t* __restrict__ bits, int64_t n, int c,
                                                       int h_in, int w_in, int h_out, int w_out, int k, int st,
                                                       int pd, int cwp, TOut* __restrict__ y,
                                                       uint32_t* __restrict__ out_bits) {
  const int64_t hwo = (int64_t)h_out * w_out;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * hwo) return;
  const int64_t frame = i / hwo;
  const int q = (int)(i - frame * hwo);
  const int oh = q / w_out, ow = q - (q / w_out) * w_out;
  uint32_t w[kSpikePoolMaxWords];
#pragma unroll
  for (int j = 0; j < kSpikePoolMaxWords; ++j) w[j] = 0u;
  const uint32_t* __restrict__ fb = bits + frame * h_in * w_in * cwp;
  for (int kh = 0; kh < k; ++kh) {
    const int ih = oh * st - pd + kh;
    if (ih < 0 || ih >= h_in) continue;
    for (int kw = 0; kw < k; ++kw) {
      const int iw = ow * st - pd + kw;
      if (iw < 0 || iw >= w_in) continue;
      const uint32_t* __restrict__ src = fb + ((int64_t)ih * w_in + iw) * cwp;
#pragma unroll
      for (int j = 0; j < kSpikePoolMaxWords; ++j)
        if (j < cwp) w[j] |= src[j];
    }
  }
  uint32_t* __restrict__ ob = out_bits + i * cwp;
#pragma unroll
  for (int j = 0; j < kSpikePoolMaxWords; ++j)
    if (j < cwp) ob[j] = w[j];
  TOut* __restrict__ yp = y + frame * c * hwo + q;
#pragma unroll
  for (int j = 0; j < kSpikePoolMaxWords; ++j) {
    if (j < cwp) {
      const uint32_t wv = w[j];
      for (int b = 0; b < 32 && 32 * j + b < c; ++b)
        yp[(int64_t)(32 * j + b) * hwo] = from_f32<TOut>((float)((wv >> b) & 1u));
    }
  }
}

}  // namespace

int launch_spike_maxpool(const uint32_t* bits, int64_t n, int c, int h_in, int w_in, int h_out, int w_out, int k,
                         int st, int pd, int cwp, int out_dtype, void* y, uint32_t* out_bits, hipStream_t stream) {
  const int64_t total = n * (int64_t)h_out * w_out;
  const int64_t blocks = (total + 255) / 256;
  if (out_dtype == SF_F16)
    hipLaunchKernelGGL(k_spike_maxpool<__half>, dim3((unsigned)blocks), dim3(256), 0, stream, bits, n, c, h_in, w_in,
                       h_out, w_out, k, st, pd, cwp, static_cast<__half*>(y), out_bits);
  else if (out_dtype == SF_BF16)
    hipLaunchKernelGGL(k_spike_maxpool<__hip_bfloat16>, dim3((unsigned)blocks), dim3(256), 0, stream, bits, n, c,
                       h_in, w_in, h_out, w_out, k, st, pd, cwp, static_cast<__hip_bfloat16*>(y), out_bits);
  else
    hipLaunchKernelGGL(k_spike_maxpool<float>, dim3((unsigned)blocks), dim3(256), 0, stream, bits, n, c, h_in, w_in,
                       h_out, w_out, k, st, pd, cwp, static_cast<float*>(y), out_bits);
  return (int)hipGetLastError();
}

}  // namespace sf
