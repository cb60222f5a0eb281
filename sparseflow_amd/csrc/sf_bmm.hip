// Spike-sparse batched matmul: C[b] = A[b] @ B[b] with A [batches, m, k]
// sparse (spike-derived queries, attention scores) and B [batches, k, n]
// dense, B read through strides so that a transposed view (K^T of
// attention) needs no copy.
//
// One workgroup (4 wavefronts) takes one (batch, column block) item: B's
// block of columns n0 .. n0+nb-1 is staged in LDS as f32 (rows padded by
// one float so that a transposed staging writes spread over the banks),
// then each wavefront takes rows of A.  A row is read 64 elements per load
// (coalesced); a ballot of |a| >= cutoff gives the segment's active
// elements as a wave-uniform mask, and the wavefront walks its set bits in
// increasing k: the element is broadcast from the lane that loaded it
// (readlane) and every lane adds it times B's row k at its columns.  Zero
// elements cost nothing; an all-zero row is just its store.  The row's
// outputs leave as coalesced runs of n, times alpha (the attention scale).
// Accumulation is f32 in increasing k: deterministic.
//
// Replaces the reference's _prescan_bmm_kernel + sparse BMM kernels
// (Kernels/bmm.py:66-184) behind sparse_bmm_forward (Kernels/bmm.py:195).
#include "sf_tile.h"

namespace sf {

namespace {

constexpr int kBmmWaves = 4;

template <typename T, typename TOut, int NBJ>
__global__ __launch_bounds__(64 * kBmmWaves) void k_bmm(BmmArgs a) {
  extern __shared__ float sb[];  // [k][nb + 1]
  constexpr int NB = 64 * NBJ;
  constexpr int LD = NB + 1;
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const T* __restrict__ A = static_cast<const T*>(a.a);
  const T* __restrict__ B = static_cast<const T*>(a.b);
  TOut* __restrict__ C = static_cast<TOut*>(a.c);
  const int K = a.k, N = a.n, M = a.m;
  const int nseg = (K + 63) / 64;
  const int64_t items = a.batches * (int64_t)a.ncb;
  for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
    const int64_t bt = item / a.ncb;
    const int n0 = (int)(item - bt * a.ncb) * NB;
    const int nbw = min(NB, N - n0);
    __syncthreads();  // the previous item is done with the staged block
    const T* __restrict__ Bb = B + bt * a.b_stride_batch;
    if (a.b_stride_n == 1) {
      for (int i = threadIdx.x; i < K * NB; i += 64 * kBmmWaves) {
        const int kk = i / NB, j = i - kk * NB;
        sb[kk * LD + j] = j < nbw ? to_f32<T>(Bb[(int64_t)kk * a.b_stride_k + n0 + j]) : 0.f;
      }
    } else {
      // Consecutive threads take consecutive k (the contiguous axis of a
      // transposed B).
      for (int i = threadIdx.x; i < K * NB; i += 64 * kBmmWaves) {
        const int j = i / K, kk = i - j * K;
        sb[kk * LD + j] = j < nbw ? to_f32<T>(Bb[(int64_t)kk * a.b_stride_k + (int64_t)(n0 + j) * a.b_stride_n]) : 0.f;
      }
    }
    __syncthreads();
    for (int m = wave; m < M; m += kBmmWaves) {
      const T* __restrict__ ar = A + (bt * M + m) * (int64_t)K;
      float acc[NBJ];
#pragma unroll
      for (int j = 0; j < NBJ; ++j) acc[j] = 0.f;
      float av = (lane < K) ? to_f32<T>(ar[lane]) : 0.f;
      for (int s = 0; s < nseg; ++s) {
        const float cur = av;
        if (s + 1 < nseg) {  // next segment's load in flight during this walk
          const int kn = (s + 1) * 64 + lane;
          av = kn < K ? to_f32<T>(ar[kn]) : 0.f;
        }
        uint64_t msk = __ballot(fabsf(cur) >= a.cutoff);
        const float* __restrict__ bs = sb + s * 64 * LD + lane;
        while (msk) {
          const int kb = __builtin_ctzll(msk);
          msk &= msk - 1;
          const float ak = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cur), kb));
          const float* __restrict__ br = bs + kb * LD;
#pragma unroll
          for (int j = 0; j < NBJ; ++j) acc[j] = fmaf(ak, br[64 * j], acc[j]);
        }
      }
      TOut* __restrict__ cr = C + (bt * M + m) * (int64_t)N + n0;
#pragma unroll
      for (int j = 0; j < NBJ; ++j)
        if (64 * j + lane < nbw) cr[64 * j + lane] = from_f32<TOut>(acc[j] * a.alpha);
    }
  }
}

template <typename T, typename TOut, int NBJ>
int launch_bmm_t(BmmArgs a, hipStream_t stream) {
  a.ncb = (a.n + 64 * NBJ - 1) / (64 * NBJ);
  const size_t lds = (size_t)a.k * (64 * NBJ + 1) * sizeof(float);
  const int64_t items = a.batches * (int64_t)a.ncb;
  const int64_t cap = (int64_t)num_cus() * 8;
  const int grid = (int)(items < cap ? items : cap);
  if (grid == 0) return (int)hipSuccess;
  hipLaunchKernelGGL((k_bmm<T, TOut, NBJ>), dim3(grid), dim3(64 * kBmmWaves), lds, stream, a);
  return (int)hipGetLastError();
}

template <typename T, typename TOut>
int launch_bmm_o(const BmmArgs& a, int nbj, hipStream_t stream) {
  switch (nbj) {
    case 4: return launch_bmm_t<T, TOut, 4>(a, stream);
    case 2: return launch_bmm_t<T, TOut, 2>(a, stream);
    default: return launch_bmm_t<T, TOut, 1>(a, stream);
  }
}

template <typename T>
int launch_bmm_d(const BmmArgs& a, int nbj, int out_dtype, hipStream_t stream) {
  if (out_dtype == SF_F32) return launch_bmm_o<T, float>(a, nbj, stream);
  return launch_bmm_o<T, T>(a, nbj, stream);
}

}  // namespace

int bmm_column_blocks(int k, int n) {
  // Widest block (up to 256 columns, never wider than n needs) whose staged
  // f32 rows fit the LDS budget of one workgroup.
  int nbj = (n + 63) / 64;
  nbj = nbj >= 4 ? 4 : (nbj >= 2 ? 2 : 1);
  while (nbj > 1 && (size_t)k * (64 * nbj + 1) * sizeof(float) > (size_t)kBmmLdsBytes) nbj >>= 1;
  if ((size_t)k * (64 * nbj + 1) * sizeof(float) > (size_t)kBmmLdsBytes) return 0;
  return nbj;
}

int launch_bmm(const BmmArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  const int nbj = bmm_column_blocks(a.k, a.n);
  timing_begin(K_BMM, stream);
  const int rc = in_dtype == SF_F16    ? launch_bmm_d<__half>(a, nbj, out_dtype, stream)
                 : in_dtype == SF_BF16 ? launch_bmm_d<__hip_bfloat16>(a, nbj, out_dtype, stream)
                                       : launch_bmm_d<float>(a, nbj, out_dtype, stream);
  timing_end(K_BMM, stream);
  return rc;
}

}  // namespace sf
