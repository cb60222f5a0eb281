// Fused spike-driven self-attention core (no softmax):
//   y[tb, m, h, :] = scale * sum_d q[tb, m, h, d] * KV[tb, h, d, :],
//   KV[tb, h, d, e] = sum_j k[tb, j, h, d] * v[tb, j, h, e]
// which equals (q @ k^T * scale) @ v of the reference's attention stages
// (Kernels/attention.py:27-121 over Kernels/bmm.py) without the seq x seq
// score matrix: per (frame, head) the kernel reads q, k and v once and
// writes y once.
//
// One workgroup (8 wavefronts) per (frame, head) item.  k and v are staged
// in LDS as f32, KV (d x d, rows padded by one float) is formed from them
// skipping zero k elements, then each wavefront takes rows of q: 64 / D rows
// per pass, lane = (row, output column e).  A ballot of the row's
// |q| >= cutoff gives its active d's; the lanes of each row walk them,
// fetch q's value from the lane that loaded it, and add it times KV's row d.
// q elements below the activity cutoff count as zero (the reference's
// prescan test on the left operand); everything is summed in f32 in
// increasing j / d order: deterministic.
//
// Layout: element (tb, m, h, d) at tb*s_tb + m*s_m + h*s_h + d for q, k, v
// (one set of strides) and for y (its own), so both token-major
// [TB, S, H, D] (the projections' output) and head-major [TB, H, S, D]
// tensors are read in place.
#include "sf_tile.h"

namespace sf {

namespace {

constexpr int kAttnThreads = 512;
constexpr int kAttnWaves = kAttnThreads / 64;

template <typename T, typename TOut, int D>
__global__ __launch_bounds__(kAttnThreads) void k_spike_attn(AttnArgs a) {
  extern __shared__ float smem[];
  constexpr int LDK = D + 1;              // padded KV row
  constexpr int EPT = D * D / kAttnThreads > 0 ? D * D / kAttnThreads : 1;
  constexpr int TPR = D / EPT;            // threads per KV row
  constexpr int R = 64 / D;               // q rows per wavefront pass
  const int S = a.s;
  float* sk = smem;
  float* sv = sk + S * D;
  float* skv = sv + S * D;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid >> 6;
  const T* __restrict__ Q = static_cast<const T*>(a.q);
  const T* __restrict__ K = static_cast<const T*>(a.k);
  const T* __restrict__ V = static_cast<const T*>(a.v);
  TOut* __restrict__ Y = static_cast<TOut*>(a.y);
  const int64_t items = a.tb * (int64_t)a.h;
  for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
    const int64_t tbi = item / a.h;
    const int hh = (int)(item - tbi * a.h);
    const int64_t base = tbi * a.s_tb + hh * a.s_h;
    const int64_t ybase = tbi * a.y_tb + hh * a.y_h;
    __syncthreads();  // the previous item is done with the staged k, v, KV
    for (int i0 = tid; i0 < S * D; i0 += 4 * kAttnThreads) {  // 8 loads in flight per thread
      float kk[4], vv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * kAttnThreads;
        const int j = i / D, dd = i - j * D;
        const int64_t off = base + (int64_t)j * a.s_m + dd;
        kk[u] = i < S * D ? to_f32<T>(K[off]) : 0.f;
        vv[u] = i < S * D ? to_f32<T>(V[off]) : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * kAttnThreads;
        if (i < S * D) {
          sk[i] = kk[u];
          sv[i] = vv[u];
        }
      }
    }
    __syncthreads();
    if (tid < D * TPR) {
      // Eight j's per step: their LDS reads are issued together.  Zero k
      // elements add exact zeros.
      const int dd = tid / TPR, e0 = (tid - dd * TPR) * EPT;
      float acc[EPT];
#pragma unroll
      for (int e = 0; e < EPT; ++e) acc[e] = 0.f;
      int j = 0;
      for (; j + 8 <= S; j += 8) {
        float kk[8], vv[8][EPT];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          kk[u] = sk[(j + u) * D + dd];
#pragma unroll
          for (int e = 0; e < EPT; ++e) vv[u][e] = sv[(j + u) * D + e0 + e];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
          for (int e = 0; e < EPT; ++e) acc[e] = fmaf(kk[u], vv[u][e], acc[e]);
      }
      for (; j < S; ++j) {
        const float kv = sk[j * D + dd];
#pragma unroll
        for (int e = 0; e < EPT; ++e) acc[e] = fmaf(kv, sv[j * D + e0 + e], acc[e]);
      }
#pragma unroll
      for (int e = 0; e < EPT; ++e) skv[dd * LDK + e0 + e] = acc[e];
    }
    __syncthreads();
    const int r = lane / D, e = lane - r * D;
    const uint64_t row_bits = D == 64 ? ~0ull : ((1ull << D) - 1ull);
    int m = wave * R + r;
    float qv = m < S ? to_f32<T>(Q[base + (int64_t)m * a.s_m + e]) : 0.f;
    for (int m0 = wave * R; m0 < S; m0 += kAttnWaves * R) {
      const float cur = qv;
      const int mn = m + kAttnWaves * R;
      if (m0 + kAttnWaves * R < S) qv = mn < S ? to_f32<T>(Q[base + (int64_t)mn * a.s_m + e]) : 0.f;
      const uint64_t bal = __ballot(fabsf(cur) >= a.cutoff);
      uint64_t msk = (bal >> (r * D)) & row_bits;
      float acc = 0.f;
      while (msk) {
        const int dd = __builtin_ctzll(msk);
        msk &= msk - 1;
        const float qd = __shfl(cur, r * D + dd, 64);
        acc = fmaf(qd, skv[dd * LDK + e], acc);
      }
      if (m < S) Y[ybase + (int64_t)m * a.y_m + e] = from_f32<TOut>(acc * a.scale);
      m = mn;
    }
  }
}

template <typename T, typename TOut, int D>
int launch_attn_t(const AttnArgs& a, hipStream_t stream) {
  const size_t lds = attn_lds_bytes(a.s, D);
  const int64_t items = a.tb * (int64_t)a.h;
  const int64_t cap = (int64_t)num_cus() * 16;
  const int grid = (int)(items < cap ? items : cap);
  if (grid == 0) return (int)hipSuccess;
  constexpr auto kern = k_spike_attn<T, TOut, D>;
  const int e = set_lds_limit_once<kern>(kMaxLdsBytes);
  if (e != (int)hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kAttnThreads), lds, stream, a);
  return (int)hipGetLastError();
}

template <typename T, typename TOut>
int launch_attn_o(const AttnArgs& a, hipStream_t stream) {
  switch (a.d) {
    case 16: return launch_attn_t<T, TOut, 16>(a, stream);
    case 32: return launch_attn_t<T, TOut, 32>(a, stream);
    default: return launch_attn_t<T, TOut, 64>(a, stream);
  }
}

template <typename T>
int launch_attn_d(const AttnArgs& a, int out_dtype, hipStream_t stream) {
  if (out_dtype == SF_F32) return launch_attn_o<T, float>(a, stream);
  return launch_attn_o<T, T>(a, stream);
}

}  // namespace

size_t attn_lds_bytes(int s, int d) { return ((size_t)2 * s * d + (size_t)d * (d + 1)) * sizeof(float); }

int launch_spike_attn(const AttnArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  timing_begin(K_ATTN, stream);
  const int rc = in_dtype == SF_F16    ? launch_attn_d<__half>(a, out_dtype, stream)
                 : in_dtype == SF_BF16 ? launch_attn_d<__hip_bfloat16>(a, out_dtype, stream)
                                       : launch_attn_d<float>(a, out_dtype, stream);
  timing_end(K_ATTN, stream);
  return rc;
}

}  // namespace sf
