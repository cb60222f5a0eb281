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
// p ~ 0.1 with head_dim 32, the seq x seq scores).  Persistent workgroups of
// four wavefronts, as many as fit on the chip, each taking batches in turn:
//  * B (k <= 256, n <= 256) is staged in LDS as bf16 hi + lo parts,
//    [n][kp] with k contiguous (rows padded, pieces XOR-swizzled: see
//    bm_row / bm_pos for the bank-conflict measurement).  A thread converts
//    one 16-byte piece (8 consecutive k of one column) at a time and writes
//    it with one ds_write_b128; pieces are handed out so that the global
//    reads are coalesced along whichever axis of B is contiguous, and
//    sixteen consecutive pieces land on distinct banks either way.
//  * Each wavefront takes 16-row tiles of A (row-major, k contiguous).  The
//    tile's whole K range is loaded into registers, split into bf16 hi + lo,
//    and the NEXT tile of the wavefront's sequence (possibly in its next
//    batch) is requested before the current one's MFMAs and stores, so that
//    HBM reads stay in flight throughout.
//  * Every 16-column tile of C takes 16x16x32 MFMAs: ah.bh + ah.bl + al.bh
//    (~16 significant bits of both operands), the ah.bl term dropped when
//    all of the batch's B is exact in bf16 and al.bh when all of the tile's
//    A is (binary spikes, small counts): both are then exact zeros.
// A elements below the activity cutoff count as zero.
// ---------------------------------------------------------------------------

namespace sf {

namespace {

typedef __bf16 bmm_bf16x8 __attribute__((ext_vector_type(8)));
typedef float bmm_f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBmKsMax = 8;  // kp <= 256
constexpr int kBmWaves = 4;

typedef __bf16 bmm_bf16x2 __attribute__((ext_vector_type(2)));
typedef float bmm_f32x2 __attribute__((ext_vector_type(2)));

// bf16 hi parts (round to nearest even) of two floats and the bf16 of their
// remainders, one packed convert each.
__device__ __forceinline__ void bm_split2(float x0, float x1, bmm_bf16x2& h, bmm_bf16x2& l) {
  const bmm_f32x2 x = {x0, x1};
  h = __builtin_convertvector(x, bmm_bf16x2);
  const bmm_f32x2 hf = __builtin_convertvector(h, bmm_f32x2);
  l = __builtin_convertvector(x - hf, bmm_bf16x2);
}

// Eight floats to bf16x8 hi and lo operands.
__device__ __forceinline__ void bm_split8(const float (&v)[8], bmm_bf16x8& h, bmm_bf16x8& l) {
  bmm_bf16x2 h0, h1, h2, h3, l0, l1, l2, l3;
  bm_split2(v[0], v[1], h0, l0);
  bm_split2(v[2], v[3], h1, l1);
  bm_split2(v[4], v[5], h2, l2);
  bm_split2(v[6], v[7], h3, l3);
  h = __builtin_shufflevector(__builtin_shufflevector(h0, h1, 0, 1, 2, 3), __builtin_shufflevector(h2, h3, 0, 1, 2, 3),
                              0, 1, 2, 3, 4, 5, 6, 7);
  l = __builtin_shufflevector(__builtin_shufflevector(l0, l1, 0, 1, 2, 3), __builtin_shufflevector(l2, l3, 0, 1, 2, 3),
                              0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ bool bm_nonzero(const bmm_bf16x8& v) {
  uint4 u;
  __builtin_memcpy(&u, &v, 16);
  return (u.x | u.y | u.z | u.w) != 0;
}

// Staged B rows: kp = 32 KS bf16, padded by one 64-byte group when KS is
// even.  Measured on gfx950 (rocprofv3 SQ_LDS_BANK_CONFLICT over
// ds_read_b128 / ds_write_b128 patterns), 16-lane fragments over rows whose
// stride is an odd number of 64-byte groups, with the 16-byte pieces of
// each group XOR-swizzled by (r >> 1) & 3, read and write without bank
// conflicts; even strides, or the swizzle by (r >> 2) & 3, do not.
template <int KS>
constexpr int bm_row() { return KS * 32 + (KS % 2 == 0 ? 32 : 0); }

// Position (bf16 elements) of element k of row r.
template <int KS>
__device__ __forceinline__ int bm_pos(int r, int k) {
  const int piece = k >> 3;
  const int sw = (piece & ~3) | ((piece & 3) ^ ((r >> 1) & 3));
  return r * bm_row<KS>() + sw * 8 + (k & 7);
}

// C tile rows in LDS: n floats padded to an odd number of 16-byte pieces
// (n % 4 == 0), which the same measurement shows conflict-free for the
// tile's 16-byte writes.
__host__ __device__ constexpr int bm_c_row(int n) { return ((n >> 2) & 1) ? n : n + 4; }

// Stage batch bt's B into s_bh / s_bl.  Returns nonzero in some thread when
// any lo part is nonzero (the caller reduces it over the workgroup).
template <typename T, int KS>
__device__ __forceinline__ uint32_t bm_stage_b(const BmmArgs& a, int64_t bt, int npad, uint16_t* s_bh,
                                               uint16_t* s_bl) {
  constexpr int kPc = KS * 4;  // 8-element pieces per column
  constexpr int kUnroll = 4;
  const T* __restrict__ Bb = static_cast<const T*>(a.b) + bt * a.b_stride_batch;
  const int K = a.k, N = a.n;
  const int npieces = npad * kPc;
  // k contiguous (a transposed view): consecutive threads take consecutive
  // pieces of one column; else consecutive columns of one piece row.
  const bool kfast = a.b_stride_k == 1 && a.b_stride_n != 1;
  const bool vec4 = kfast && sizeof(T) == 4 && (a.b_stride_n & 3) == 0 && (a.b_stride_batch & 3) == 0 &&
                    (reinterpret_cast<uintptr_t>(a.b) & 15) == 0;
  uint32_t lo_any = 0;
  const int tid = threadIdx.x;
  for (int p0 = tid; p0 < npieces; p0 += 64 * kBmWaves * kUnroll) {
    float v[kUnroll][8];
    int col[kUnroll], pc[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int p = p0 + 64 * kBmWaves * u;
      int nn, c;
      if (kfast) {
        nn = p / kPc;
        c = p - nn * kPc;
      } else {
        c = p / npad;
        nn = p - c * npad;
      }
      col[u] = p < npieces ? nn : -1;
      pc[u] = c;
      const int k0 = c * 8;
      const bool colok = p < npieces && nn < N;
      if (vec4 && colok && k0 + 8 <= K) {
        const float4* src = reinterpret_cast<const float4*>(Bb + (int64_t)nn * a.b_stride_n + k0);
        const float4 t0 = src[0], t1 = src[1];
        v[u][0] = t0.x; v[u][1] = t0.y; v[u][2] = t0.z; v[u][3] = t0.w;
        v[u][4] = t1.x; v[u][5] = t1.y; v[u][6] = t1.z; v[u][7] = t1.w;
      } else {
        // Clamped in-bounds reads, masked after: no per-element branches.
        const int nc = nn < N ? nn : N - 1;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int kc = k0 + j < K ? k0 + j : K - 1;
          const float x = to_f32<T>(Bb[(int64_t)kc * a.b_stride_k + (int64_t)nc * a.b_stride_n]);
          v[u][j] = (colok && k0 + j < K) ? x : 0.f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (col[u] < 0) continue;
      bmm_bf16x8 h, l;
      bm_split8(v[u], h, l);
      lo_any |= bm_nonzero(l) ? 1u : 0u;
      const int pos = bm_pos<KS>(col[u], pc[u] * 8);
      *reinterpret_cast<bmm_bf16x8*>(&s_bh[pos]) = h;
      *reinterpret_cast<bmm_bf16x8*>(&s_bl[pos]) = l;
    }
  }
  return lo_any;
}

// Raw A values of one 16-row tile: lane (li, g) holds row 16 mt + li,
// k = 32 ks + 8 g .. +7.  Rows past m are not read.
template <typename T, int KS>
__device__ __forceinline__ void bm_load_a(float (&av)[KS][8], const BmmArgs& a, int64_t bt, int mt, bool vec) {
  const int li = lane_id() & 15, g = lane_id() >> 4;
  const int row = mt * 16 + li;
  const int K = a.k;
  if (row >= a.m) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) av[ks][j] = 0.f;
    return;
  }
  const T* __restrict__ ar = static_cast<const T*>(a.a) + (bt * a.m + row) * (int64_t)K;
  if (vec) {  // K % 4 == 0: whole float4 groups are in or out
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k0 = ks * 32 + 8 * g + 4 * h;
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        // KS = ceil(K / 32): only the last slice can reach past K.
        if (ks < KS - 1 || k0 < K) t = *reinterpret_cast<const float4*>(ar + k0);
        av[ks][4 * h] = t.x; av[ks][4 * h + 1] = t.y; av[ks][4 * h + 2] = t.z; av[ks][4 * h + 3] = t.w;
      }
  } else {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int k = ks * 32 + 8 * g + j;
        const bool in = ks < KS - 1 || k < K;
        const float x = to_f32<T>(ar[in ? k : K - 1]);
        av[ks][j] = in ? x : 0.f;
      }
  }
}

// Four consecutive outputs of one row, one vector store when `vec`.
template <typename TOut>
__device__ __forceinline__ void bm_store4(TOut* p, const bmm_f32x4& v, float alpha, int nvalid, bool vec) {
  if (vec && nvalid >= 4) {
    if constexpr (sizeof(TOut) == 4) {
      *reinterpret_cast<float4*>(p) = make_float4(v[0] * alpha, v[1] * alpha, v[2] * alpha, v[3] * alpha);
    } else {
      TOut h[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) h[i] = from_f32<TOut>(v[i] * alpha);
      uint2 u;
      __builtin_memcpy(&u, h, 8);
      *reinterpret_cast<uint2*>(p) = u;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (i < nvalid) p[i] = from_f32<TOut>(v[i] * alpha);
  }
}

// C tile (mt, every column tile) from the split A tile and the staged B.
// The MFMAs compute the transposed tile, D[n][m] = sum_k B[k][n] A[m][k]
// (B's staged [n][k] pieces are the first operand, A's registers the
// second), so that lane (li, g) ends with row 16 mt + li, columns
// 16 nt + 4 g .. +3 of C.  With s_c (n % 4 == 0) the wavefront collects
// the tile's rows in LDS (rows of bm_c_row(n) floats) and copies them out
// as the one contiguous block of rows x n values they form in C, in 16-byte
// pieces: whole cache lines per store instead of 64-byte pieces of sixteen
// rows.  Else each lane stores its four outputs directly.
// blo / alo (wave-uniform): B / the A tile has nonzero lo parts.
template <typename TOut, int KS>
__device__ __forceinline__ void bm_tile(const bmm_bf16x8 (&ah)[KS], const bmm_bf16x8 (&al)[KS],
                                        const uint16_t* s_bh, const uint16_t* s_bl, float* s_c, const BmmArgs& a,
                                        int64_t bt, int mt, int ntiles, bool blo, bool alo, bool vec_out) {
  const int lane = lane_id(), li = lane & 15, g = lane >> 4;
  const int row = mt * 16 + li;
  TOut* __restrict__ cr = static_cast<TOut*>(a.c) + (bt * a.m + (row < a.m ? row : 0)) * (int64_t)a.n + 4 * g;
  // bm_pos(col, 32 ks + 8 g): the lane's piece within each 64-byte group is
  // g ^ ((col >> 1) & 3), the same for every ks and every column tile
  // (col advances by 16), so one base per array and immediate offsets.
  const int lbase = li * bm_row<KS>() + 8 * (g ^ ((li >> 1) & 3));
  const bmm_bf16x8* __restrict__ ph = reinterpret_cast<const bmm_bf16x8*>(s_bh + lbase);
  const bmm_bf16x8* __restrict__ pl = reinterpret_cast<const bmm_bf16x8*>(s_bl + lbase);
#pragma clang loop unroll(disable)
  for (int nt = 0; nt < ntiles; ++nt) {
    bmm_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const bmm_bf16x8 bh = ph[ks * 4];  // 32 bf16 per ks
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh, ah[ks], acc, 0, 0, 0);
      if (blo) {
        const bmm_bf16x8 bl = pl[ks * 4];
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bl, ah[ks], acc, 0, 0, 0);
      }
      if (alo) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh, al[ks], acc, 0, 0, 0);
    }
    ph += 16 * bm_row<KS>() / 8;  // 16 rows of staged B
    pl += 16 * bm_row<KS>() / 8;
    const int c0 = nt * 16 + 4 * g;
    if (s_c != nullptr) {
      if (c0 < a.n) *reinterpret_cast<bmm_f32x4*>(s_c + li * bm_c_row(a.n) + c0) = acc;
    } else if (row < a.m) {
      bm_store4<TOut>(cr + nt * 16, acc, a.alpha, a.n - c0, vec_out);
    }
  }
  if (s_c != nullptr) {
    const int rows = a.m - mt * 16 < 16 ? a.m - mt * 16 : 16;
    const int total = rows * a.n;  // a multiple of 4
    TOut* __restrict__ cb = static_cast<TOut*>(a.c) + (bt * a.m + mt * 16) * (int64_t)a.n;
    const int crow = bm_c_row(a.n);
    // r = e / n: e < 4096 and n <= 256 keep (e + 0.5) / n at least 1 / 512
    // away from an integer, far beyond the rounding of the product.
    const float inv_n = 1.f / (float)a.n;
    for (int e = lane * 4; e < total; e += 256) {
      const int r = (int)(((float)e + 0.5f) * inv_n), c = e - r * a.n;
      bm_store4<TOut>(cb + e, *reinterpret_cast<const bmm_f32x4*>(s_c + r * crow + c), a.alpha, 4, true);
    }
  }
}

// stage_c: each wavefront also has a 16 x n f32 C tile in LDS after B
// (n % 4 == 0, C rows 16-byte aligned).
template <typename T, typename TOut, int KS>
__global__ __launch_bounds__(64 * kBmWaves) __attribute__((amdgpu_waves_per_eu(KS <= 7 ? 3 : 2)))
void k_bmm_mfma(BmmArgs a, int stage_c) {
  extern __shared__ __align__(16) uint16_t s_b[];  // hi [npad][bm_row], lo, then C tiles
  const int npad = (a.n + 15) & ~15;
  uint16_t* s_bh = s_b;
  uint16_t* s_bl = s_b + npad * bm_row<KS>();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int mtiles = (a.m + 15) / 16, ntiles = npad / 16;
  // f32 rows of A 16-byte aligned: rows start at multiples of K floats.
  const bool vec = sizeof(T) == 4 && (a.k & 3) == 0 && (reinterpret_cast<uintptr_t>(a.a) & 15) == 0;
  const bool has_tiles = wave < mtiles;
  float* s_c = stage_c ? reinterpret_cast<float*>(s_b + 2 * npad * bm_row<KS>()) + wave * 16 * bm_c_row(a.n) : nullptr;
  // Rows of C start 4-element aligned: four outputs leave as one store.
  const bool vec_out = (a.n & 3) == 0 && (reinterpret_cast<uintptr_t>(a.c) & (4 * sizeof(TOut) - 1)) == 0;
  // This wavefront's items, in order: tiles wave, wave + 4, ... of batch
  // blockIdx.x, then of batch blockIdx.x + gridDim.x, ...  av holds the raw
  // A of the next item to compute.
  float av[KS][8];
  int64_t nb = blockIdx.x;
  int nm = wave;
  if (has_tiles && nb < a.batches) bm_load_a<T, KS>(av, a, nb, nm, vec);
  for (int64_t bt = blockIdx.x; bt < a.batches; bt += gridDim.x) {
    __syncthreads();  // the previous batch is done with s_b
    const uint32_t blo = __syncthreads_or((int)bm_stage_b<T, KS>(a, bt, npad, s_bh, s_bl));
    if (!has_tiles) continue;
    for (int mt = wave; mt < mtiles; mt += kBmWaves) {
      bmm_bf16x8 ah[KS], al[KS];
      bool alo = false;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int j = 0; j < 8; ++j) av[ks][j] = fabsf(av[ks][j]) >= a.cutoff ? av[ks][j] : 0.f;
        bm_split8(av[ks], ah[ks], al[ks]);
        alo |= bm_nonzero(al[ks]);
      }
      // Request the next item's A before this tile's MFMAs and stores.
      nm += kBmWaves;
      if (nm >= mtiles) {
        nm = wave;
        nb += gridDim.x;
      }
      if (nb < a.batches) bm_load_a<T, KS>(av, a, nb, nm, vec);
      const bool any_alo = __builtin_amdgcn_ballot_w64(alo) != 0;
      bm_tile<TOut, KS>(ah, al, s_bh, s_bl, s_c, a, bt, mt, ntiles, blo != 0, any_alo, vec_out);
    }
  }
}

// Workgroups of k_bmm_mfma<...> that fit on one CU with `lds` bytes of
// dynamic LDS each (cached per kernel, device and size).
template <auto K>
int bm_blocks_per_cu(size_t lds) {
  static std::atomic<uint64_t> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  std::atomic<uint64_t>& slot = cache[dev & 63];
  const uint64_t c = slot.load(std::memory_order_relaxed);
  if (c != 0 && (c >> 8) == lds) return (int)(c & 0xff);
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, reinterpret_cast<const void*>(K), 64 * kBmWaves, lds) !=
          hipSuccess ||
      blocks <= 0)
    blocks = 1;
  if (blocks > 255) blocks = 255;
  slot.store(((uint64_t)lds << 8) | (uint64_t)blocks, std::memory_order_relaxed);
  return blocks;
}

template <typename T, typename TOut, int KS>
int launch_bmm_mfma_t(const BmmArgs& a, hipStream_t stream) {
  const size_t lds_b = (size_t)2 * ((a.n + 15) & ~15) * bm_row<KS>() * sizeof(uint16_t);
  const size_t lds_c = (size_t)kBmWaves * 16 * bm_c_row(a.n) * sizeof(float);
  // Stage C tiles when rows are whole 16-byte pieces and two workgroups
  // still fit on a CU.
  const bool vec_out = (a.n & 3) == 0 && (reinterpret_cast<uintptr_t>(a.c) & (4 * sizeof(TOut) - 1)) == 0;
  const int stage_c = vec_out && lds_b + lds_c <= (size_t)80 * 1024 ? 1 : 0;
  const size_t lds = lds_b + (stage_c ? lds_c : 0);
  constexpr auto kern = k_bmm_mfma<T, TOut, KS>;
  // Beyond the default 64 KB: padded B rows of the widest shapes (at most
  // 1.5 x 64 KB, KS = 2) or B plus C tiles (at most 80 KB).
  if (lds > 64 * 1024) {
    const int e = set_lds_limit_once<kern>(96 * 1024);
    if (e != (int)hipSuccess) return e;
  }
  const int64_t cap = (int64_t)num_cus() * bm_blocks_per_cu<kern>(lds);
  const int grid = (int)(a.batches < cap ? a.batches : cap);
  if (grid == 0) return (int)hipSuccess;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * kBmWaves), lds, stream, a, stage_c);
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
