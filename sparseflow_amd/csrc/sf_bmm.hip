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
    // Unrolled so that eight global loads are in flight per thread (the LDS
    // stores do not alias them).
    if (a.b_stride_n == 1) {
#pragma unroll 8
      for (int i = threadIdx.x; i < K * NB; i += 64 * kBmmWaves) {
        const int kk = i / NB, j = i - kk * NB;
        sb[kk * LD + j] = j < nbw ? to_f32<T>(Bb[(int64_t)kk * a.b_stride_k + n0 + j]) : 0.f;
      }
    } else {
      // Consecutive threads take consecutive k (the contiguous axis of a
      // transposed B).
#pragma unroll 8
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

// ---------------------------------------------------------------------------
// Batched matmul on the matrix cores, for the attention shapes (A's rows
// dense enough that every 32-wide K slice of a 16-row tile is live: q at
// p ~ 0.1 with head_dim 32, the seq x seq scores).  One workgroup per batch:
// B (k <= 256, n <= 256) is converted to bf16 hi + lo parts into LDS,
// [n][kp] with k contiguous and an XOR piece swizzle; each wavefront takes
// 16-row tiles of A, loads the tile's whole K range from HBM once, splits it
// into bf16 hi + lo in registers, and computes every 16-column tile of C
// with 16x16x32 MFMAs (ah.bh + ah.bl + al.bh: ~16 bits of both operands).
// A elements below the activity cutoff count as zero.
// ---------------------------------------------------------------------------

namespace sf {

namespace {

typedef __bf16 bmm_bf16x8 __attribute__((ext_vector_type(8)));
typedef float bmm_f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBmKsMax = 8;  // kp <= 256

__device__ __forceinline__ uint16_t bm_bf16_bits(float f) {
  const __hip_bfloat16 h = __float2bfloat16(f);
  uint16_t u;
  __builtin_memcpy(&u, &h, 2);
  return u;
}

// Position (bf16 elements) of element k of row r in a [rows][kp] tile whose
// 16-byte pieces are XOR-swizzled within each 64-byte group by (r >> 2) & 3.
__device__ __forceinline__ int bm_pos(int r, int k, int kp) {
  const int piece = k >> 3;
  const int sw = (piece & ~3) | ((piece & 3) ^ ((r >> 2) & 3));
  return r * kp + sw * 8 + (k & 7);
}

template <typename T, typename TOut, int KS>
__global__ __launch_bounds__(256) void k_bmm_mfma(BmmArgs a) {
  extern __shared__ __align__(16) uint16_t s_b[];  // hi [npad][kp], then lo
  const int kp = KS * 32;
  const int npad = (a.n + 15) & ~15;
  uint16_t* s_bh = s_b;
  uint16_t* s_bl = s_b + npad * kp;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  const T* __restrict__ A = static_cast<const T*>(a.a);
  const T* __restrict__ B = static_cast<const T*>(a.b);
  TOut* __restrict__ C = static_cast<TOut*>(a.c);
  const int M = a.m, K = a.k, N = a.n;
  const int mtiles = (M + 15) / 16, ntiles = npad / 16;
  // f32 rows of A 16-byte aligned: rows start at multiples of K floats.
  const bool vec = sizeof(T) == 4 && (K & 3) == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0;
  for (int64_t bt = blockIdx.x; bt < a.batches; bt += gridDim.x) {
    __syncthreads();  // the previous batch is done with s_b
    const T* __restrict__ Bb = B + bt * a.b_stride_batch;
    // Stage B: consecutive threads walk B's contiguous axis, sixteen loads in
    // flight per thread (one at a time, the staging was a chain of up to a
    // few hundred dependent global loads).
    const bool kfast = a.b_stride_k == 1 && a.b_stride_n != 1;
    const int nb = npad * kp;
    constexpr int U = 16;
    for (int i0 = tid; i0 < nb; i0 += 256 * U) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + 256 * u;
        int kk, nn;
        if (kfast) { nn = i / kp; kk = i - nn * kp; } else { kk = i / npad; nn = i - kk * npad; }
        v[u] = (i < nb && kk < K && nn < N) ? to_f32<T>(Bb[(int64_t)kk * a.b_stride_k + (int64_t)nn * a.b_stride_n])
                                            : 0.f;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + 256 * u;
        if (i < nb) {
          int kk, nn;
          if (kfast) { nn = i / kp; kk = i - nn * kp; } else { kk = i / npad; nn = i - kk * npad; }
          const uint16_t h = bm_bf16_bits(v[u]);
          const uint16_t l = bm_bf16_bits(v[u] - __uint_as_float((uint32_t)h << 16));
          const int pos = bm_pos(nn, kk, kp);
          s_bh[pos] = h;
          s_bl[pos] = l;
        }
      }
    }
    __syncthreads();
    const T* __restrict__ Ab = A + bt * (int64_t)M * K;
    TOut* __restrict__ Cb = C + bt * (int64_t)M * N;
    for (int mt = wave; mt < mtiles; mt += 4) {
      const int row = mt * 16 + li;
      const bool row_ok = row < M;
      const T* __restrict__ ar = Ab + (int64_t)(row_ok ? row : 0) * K;
      // The tile's whole K range: lane (li, g) holds k = 32 ks + 8 g .. +7.
      float av[KS][8];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int kk0 = ks * 32 + 8 * g;
        if (vec && kk0 + 8 <= K) {  // two 16-byte loads
          const float4 t0 = *reinterpret_cast<const float4*>(ar + kk0);
          const float4 t1 = *reinterpret_cast<const float4*>(ar + kk0 + 4);
          av[ks][0] = t0.x; av[ks][1] = t0.y; av[ks][2] = t0.z; av[ks][3] = t0.w;
          av[ks][4] = t1.x; av[ks][5] = t1.y; av[ks][6] = t1.z; av[ks][7] = t1.w;
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) av[ks][j] = to_f32<T>(ar[kk0 + j < K ? kk0 + j : 0]);
        }
      }
      bmm_bf16x8 ah[KS], al[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int kk = ks * 32 + 8 * g + j;
          const float v = (row_ok && kk < K && fabsf(av[ks][j]) >= a.cutoff) ? av[ks][j] : 0.f;
          const uint16_t h = bm_bf16_bits(v);
          const uint16_t l = bm_bf16_bits(v - __uint_as_float((uint32_t)h << 16));
          __bf16 hb, lb;
          __builtin_memcpy(&hb, &h, 2);
          __builtin_memcpy(&lb, &l, 2);
          ah[ks][j] = hb;
          al[ks][j] = lb;
        }
      for (int nt = 0; nt < ntiles; ++nt) {
        bmm_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const int col = nt * 16 + li;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int pos = bm_pos(col, ks * 32 + 8 * g, kp);
          const bmm_bf16x8 bh = *reinterpret_cast<const bmm_bf16x8*>(&s_bh[pos]);
          const bmm_bf16x8 bl = *reinterpret_cast<const bmm_bf16x8*>(&s_bl[pos]);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[ks], bh, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[ks], bl, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[ks], bh, acc, 0, 0, 0);
        }
        // acc element i: row 16 mt + 4 g + i, column nt * 16 + li.
        if (col < N) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = mt * 16 + 4 * g + i;
            if (r < M) Cb[(int64_t)r * N + col] = from_f32<TOut>(acc[i] * a.alpha);
          }
        }
      }
    }
  }
}

template <typename T, typename TOut, int KS>
int launch_bmm_mfma_t(const BmmArgs& a, hipStream_t stream) {
  const size_t lds = (size_t)2 * ((a.n + 15) & ~15) * (KS * 32) * sizeof(uint16_t);
  const int64_t cap = (int64_t)num_cus() * 8;
  const int grid = (int)(a.batches < cap ? a.batches : cap);
  if (grid == 0) return (int)hipSuccess;
  hipLaunchKernelGGL((k_bmm_mfma<T, TOut, KS>), dim3(grid), dim3(256), lds, stream, a);
  return (int)hipGetLastError();
}

template <typename T, typename TOut>
int launch_bmm_mfma_o(const BmmArgs& a, hipStream_t stream) {
  switch ((a.k + 31) / 32) {
    case 1: return launch_bmm_mfma_t<T, TOut, 1>(a, stream);
    case 2: return launch_bmm_mfma_t<T, TOut, 2>(a, stream);
    case 3: return launch_bmm_mfma_t<T, TOut, 3>(a, stream);
    case 4: return launch_bmm_mfma_t<T, TOut, 4>(a, stream);
    case 5: return launch_bmm_mfma_t<T, TOut, 5>(a, stream);
    case 6: return launch_bmm_mfma_t<T, TOut, 6>(a, stream);
    case 7: return launch_bmm_mfma_t<T, TOut, 7>(a, stream);
    default: return launch_bmm_mfma_t<T, TOut, 8>(a, stream);
  }
}

template <typename T>
int launch_bmm_mfma_d(const BmmArgs& a, int out_dtype, hipStream_t stream) {
  if (out_dtype == SF_F32) return launch_bmm_mfma_o<T, float>(a, stream);
  return launch_bmm_mfma_o<T, T>(a, stream);
}

}  // namespace

bool bmm_mfma_supported(int k, int n) {
  const int kp = (k + 31) / 32 * 32, npad = (n + 15) & ~15;
  return k >= 1 && n >= 1 && kp <= 32 * kBmKsMax && (int64_t)npad * kp * 2 * 2 <= kBmmLdsBytes;
}

int launch_bmm_mfma(const BmmArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  timing_begin(K_BMM_MFMA, stream);
  const int rc = in_dtype == SF_F16    ? launch_bmm_mfma_d<__half>(a, out_dtype, stream)
                 : in_dtype == SF_BF16 ? launch_bmm_mfma_d<__hip_bfloat16>(a, out_dtype, stream)
                                       : launch_bmm_mfma_d<float>(a, out_dtype, stream);
  timing_end(K_BMM_MFMA, stream);
  return rc;
}

}  // namespace sf
