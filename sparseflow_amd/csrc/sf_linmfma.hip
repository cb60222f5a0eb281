// Sparse Linear on the matrix cores: y[m, c_out] = x[m, k] @ W^T + bias at
// transformer spike densities (p ~ 0.1), where every 32-wide slice of K is
// live in some row of a tile and a VALU walk over the spikes loses to MFMA.
//
// Exactness without fp32 MFMA: W is split on the host into bf16 hi + lo
// parts (W = hi + lo + O(2^-17 |W|)) and x in the kernel (x = xh + xl; xl is
// zero for spikes and small integers), and y = xh @ hi^T + xh @ lo^T +
// xl @ hi^T carries ~16 bits of both operands.  Elements with f16(|x|) <=
// f16(threshold) count as zero, as in the prescan.
//
// One workgroup (4 wavefronts, 2 x 2) computes a 128-row x 128-column tile;
// each wavefront 64 x 64 = 4 x 4 MFMA 16x16x32 bf16 tiles (64 f32
// accumulators per lane).  K is walked in 32-wide steps: the x tile (128 x
// 32, converted to bf16 in registers) and the W tiles (128 columns x 32 of
// the [c_out][kp] bf16 hi and lo rows, from L2) are staged in LDS,
// double-buffered with one barrier per step; the next step's loads are in
// flight during the current step's MFMAs.  The main walk computes xh @ hi^T
// + xh @ lo^T and notes whether any staged element of x has a non-zero xl;
// only a workgroup that saw one walks K a second time for xl @ hi^T (for
// spikes, the transformer case, the third product is never formed).  The
// MFMAs of a walk run unconditionally: a data-dependent branch around them
// makes the compiler copy the 64 accumulators between AGPRs and VGPRs every
// step, which costs more than the products it would skip (an all-zero 128 x
// 32 slice of x is vanishingly rare at these densities; the spike walk
// serves sparse inputs).
// Row blocks are the slow index of the grid and workgroups are placed
// XCD-locally, so the column blocks of one row block run together on one
// XCD and share its x tile through that XCD's L2.
//
// Replaces the reference's sparse_linear_grouped_kernel (Kernels/linear.py:
// 360-457: fp16 tl.dot over active groups, dense tiles when all groups are
// live) for such inputs.
#include <type_traits>

#include "sf_tile.h"

namespace sf {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kLmRows = 128;        // rows per workgroup tile
constexpr int kLmCols = 128;        // output columns per workgroup tile
constexpr int kLmK = 32;            // K per step
constexpr int kLmLda = kLmK;        // LDS row: 32 bf16 = 64 B, four 16-byte pieces
// 16-byte piece p of tile row r sits at piece p ^ ((r >> 1) & 3) of its
// row.  Measured on gfx950 (rocprofv3 SQ_LDS_BANK_CONFLICT over the
// kernel's ds_read_b128 fragment reads and ds_write_b128 staging writes):
// with 64-byte rows this swizzle is conflict-free for both, while the
// swizzle by (r >> 2) & 3 -- which also covers every bank once per 16 lanes
// -- costs a third more LDS cycles on the reads and doubles the writes.
__device__ __forceinline__ int lm_piece(int r, int p) { return p ^ ((r >> 1) & 3); }
constexpr int kLmMaxK = 8192;

__device__ __forceinline__ uint16_t bf16_bits(float f) {
  const __hip_bfloat16 h = __float2bfloat16(f);  // round to nearest even
  uint16_t u;
  __builtin_memcpy(&u, &h, 2);
  return u;
}

__device__ __forceinline__ float bf16_value(uint16_t u) {
  return __uint_as_float((uint32_t)u << 16);
}

// 16 consecutive elements of row `row` from column kk0, without branches
// and without touching the loaded values: out-of-range rows and columns
// load a valid element, and the count of valid elements (0..16) is returned
// for the staging to zero the rest -- any use of the values here would make
// the compiler wait for the loads before the MFMAs they are meant to
// overlap.  VEC: f32 input, k % 16 == 0 and x 16-byte aligned, so a
// 16-element run is entirely inside or entirely past the row.
template <typename TIn, bool VEC>
__device__ __forceinline__ int lm_load_x(const TIn* __restrict__ x, int64_t m, int k, int row, int kk0,
                                         float (&v)[16]) {
  const bool row_ok = row < m;
  const int64_t rr = row_ok ? row : 0;
  const int valid = row_ok ? min(max(k - kk0, 0), 16) : 0;
  if constexpr (VEC) {
    const float4* p = reinterpret_cast<const float4*>(x + rr * k + (valid > 0 ? kk0 : 0));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 t = p[q];
      v[4 * q] = t.x;
      v[4 * q + 1] = t.y;
      v[4 * q + 2] = t.z;
      v[4 * q + 3] = t.w;
    }
  } else {
    // Raw 16-bit or 32-bit elements; converted in the staging.
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const TIn t = x[rr * k + (j < valid ? kk0 + j : 0)];
      if constexpr (sizeof(TIn) == 4) {
        v[j] = t;
      } else {
        uint16_t u;
        __builtin_memcpy(&u, &t, 2);
        v[j] = __uint_as_float((uint32_t)u);  // bit pattern carried in a float register
      }
    }
  }
  return valid;
}

template <typename TIn, bool VEC>
__device__ __forceinline__ float lm_value(float raw) {
  if constexpr (VEC || sizeof(TIn) == 4) {
    return raw;
  } else {
    const uint16_t u = (uint16_t)__float_as_uint(raw);
    TIn t;
    __builtin_memcpy(&t, &u, 2);
    return to_f32<TIn>(t);
  }
}

template <typename TIn, typename TOut, bool VEC>
__global__ __launch_bounds__(256) void k_linear_mfma(LinMfmaArgs a) {
  // Double-buffered LDS tiles (bf16 bit patterns): x [128 rows][32] (its hi
  // part in the main walk, its lo part in the second), W hi / lo [128
  // columns][32]; 48 KB.
  __shared__ __align__(16) uint16_t s_xh[2][kLmRows * kLmLda];
  __shared__ __align__(16) uint16_t s_wh[2][kLmCols * kLmLda];
  __shared__ __align__(16) uint16_t s_wl[2][kLmCols * kLmLda];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int ncb = (a.c_out + kLmCols - 1) / kLmCols;
  // The column blocks of a row block share its x tile through L2, which is
  // per XCD: placed XCD-locally, consecutive tiles run on one XCD.
  const int bid = xcd_range_block((int)blockIdx.x, (int)gridDim.x);
  const int64_t rb = bid / ncb;
  const int cb = (int)(bid - rb * ncb);
  const int64_t r0 = rb * kLmRows;
  const int c0 = cb * kLmCols;
  const int nsteps = a.kp / kLmK;
  const TIn* __restrict__ X = static_cast<const TIn*>(a.x);

  // Staging: thread t takes x row t / 2 and W column t / 2 of the tile, 16
  // k values at 16 * (t & 1).  Columns past c_out stage W row 0 (never stored).
  const int sr = tid >> 1, sh = tid & 1;
  const int wcol = c0 + sr < a.c_out ? c0 + sr : 0;
  const uint4* wh_src = reinterpret_cast<const uint4*>(a.wh + (int64_t)wcol * a.kp + 16 * sh);
  const uint4* wl_src = reinterpret_cast<const uint4*>(a.wl + (int64_t)wcol * a.kp + 16 * sh);
  float v[16];
  int v_valid = 0;
  uint4 wh0, wh1, wl0, wl1;
  // LO = false: the main walk (x hi, W hi and lo); LO = true: the second walk
  // (x lo, W hi).
  auto load_step = [&](int step, auto lo_walk) {
    constexpr bool LO = decltype(lo_walk)::value;
    const int kb = step * kLmK;  // 16-byte units: kb / 8
    wh0 = wh_src[kb / 8];
    wh1 = wh_src[kb / 8 + 1];
    if constexpr (!LO) {
      wl0 = wl_src[kb / 8];
      wl1 = wl_src[kb / 8 + 1];
    }
    v_valid = lm_load_x<TIn, VEC>(X, a.m, a.k, (int)(r0 + sr), kb + 16 * sh, v);  // r0 + sr < 2^30 + 128
  };
  bool inexact = false;  // some staged element of x has a non-zero lo part
  auto stage = [&](int buf, auto lo_walk) {
    constexpr bool LO = decltype(lo_walk)::value;
    uint32_t hx[8];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float t = lm_value<TIn, VEC>(v[j]);
      v[j] = (j < v_valid && fabsf(t) >= a.cutoff) ? t : 0.f;  // range, then the prescan's activity test
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint16_t h0 = bf16_bits(v[2 * j]), h1 = bf16_bits(v[2 * j + 1]);
      const float r0v = v[2 * j] - bf16_value(h0), r1v = v[2 * j + 1] - bf16_value(h1);
      if constexpr (LO) {
        hx[j] = (uint32_t)bf16_bits(r0v) | ((uint32_t)bf16_bits(r1v) << 16);
      } else {
        inexact |= (r0v != 0.f) | (r1v != 0.f);
        hx[j] = (uint32_t)h0 | ((uint32_t)h1 << 16);
      }
    }
    const int p0 = 8 * lm_piece(sr, 2 * sh), p1 = 8 * lm_piece(sr, 2 * sh + 1);  // bf16 offsets
    uint16_t* rx = &s_xh[buf][sr * kLmLda];
    uint16_t* rwh = &s_wh[buf][sr * kLmLda];
    *reinterpret_cast<uint4*>(rx + p0) = make_uint4(hx[0], hx[1], hx[2], hx[3]);
    *reinterpret_cast<uint4*>(rx + p1) = make_uint4(hx[4], hx[5], hx[6], hx[7]);
    *reinterpret_cast<uint4*>(rwh + p0) = wh0;
    *reinterpret_cast<uint4*>(rwh + p1) = wh1;
    if constexpr (!LO) {
      uint16_t* rwl = &s_wl[buf][sr * kLmLda];
      *reinterpret_cast<uint4*>(rwl + p0) = wl0;
      *reinterpret_cast<uint4*>(rwl + p1) = wl1;
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int g = lane >> 4, li = lane & 15;
  // One walk over K: per step, x [128 x 32] times W^T [32 x 128] as the
  // products of the staged x tile with the staged W hi (and, in the main
  // walk, W lo) tiles.
  auto walk = [&](auto lo_walk) {
    constexpr bool LO = decltype(lo_walk)::value;
    load_step(0, lo_walk);
    stage(0, lo_walk);
    __syncthreads();
    for (int step = 0; step < nsteps; ++step) {
      const int buf = step & 1;
      // Next step's tiles are in flight during this step's MFMAs; the staging
      // after them is their first use.
      if (step + 1 < nsteps) load_step(step + 1, lo_walk);
      // Keep the scheduler from pulling the staging math (which waits for
      // those loads) above the MFMAs.
      __builtin_amdgcn_sched_barrier(0);
      {
        bf16x8 ax[4], bh[4], bl[4];
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          const int r = 64 * wc + 16 * ct + li;
          const int c = r * kLmLda + 8 * lm_piece(r, g);
          bh[ct] = *reinterpret_cast<const bf16x8*>(&s_wh[buf][c]);
          if constexpr (!LO) bl[ct] = *reinterpret_cast<const bf16x8*>(&s_wl[buf][c]);
        }
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
          const int r = 64 * wr + 16 * rt + li;
          ax[rt] = *reinterpret_cast<const bf16x8*>(&s_xh[buf][r * kLmLda + 8 * lm_piece(r, g)]);
        }
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
          for (int ct = 0; ct < 4; ++ct)
            acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ax[rt], bh[ct], acc[rt][ct], 0, 0, 0);
        if constexpr (!LO) {
#pragma unroll
          for (int rt = 0; rt < 4; ++rt)
#pragma unroll
            for (int ct = 0; ct < 4; ++ct)
              acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ax[rt], bl[ct], acc[rt][ct], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (step + 1 < nsteps) stage(buf ^ 1, lo_walk);
      __syncthreads();
    }
  };
  walk(std::false_type{});
  // Every staged element's lo part was zero in every thread: done (the
  // barrier's result is the same in every wavefront, so the branch is
  // uniform).
  if (__syncthreads_or(inexact ? 1 : 0)) walk(std::true_type{});

  // Accumulator (rt, ct) element i of lane l: row 16 rt + 4 (l >> 4) + i,
  // column 16 ct + (l & 15) of the wavefront's 64 x 64 tile.
  TOut* __restrict__ Y = static_cast<TOut*>(a.y);
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const int col = c0 + 64 * wc + 16 * ct + li;
    if (col >= a.c_out) continue;
    const float b = a.bias != nullptr ? a.bias[col] : 0.f;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = r0 + 64 * wr + 16 * rt + 4 * g + i;
        if (row < a.m) Y[row * a.c_out + col] = from_f32<TOut>(acc[rt][ct][i] + b);
      }
  }
}

template <typename TIn>
int launch_lm_d(const LinMfmaArgs& a, int out_dtype, hipStream_t stream) {
  const int64_t rbs = (a.m + kLmRows - 1) / kLmRows;
  const int64_t grid = rbs * ((a.c_out + kLmCols - 1) / kLmCols);
  if (grid == 0) return (int)hipSuccess;
  const bool vec = sizeof(TIn) == 4 && a.k % 16 == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0;
  if (vec) {
    if (out_dtype == SF_F32)
      hipLaunchKernelGGL((k_linear_mfma<TIn, float, true>), dim3((unsigned)grid), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((k_linear_mfma<TIn, TIn, true>), dim3((unsigned)grid), dim3(256), 0, stream, a);
  } else {
    if (out_dtype == SF_F32)
      hipLaunchKernelGGL((k_linear_mfma<TIn, float, false>), dim3((unsigned)grid), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((k_linear_mfma<TIn, TIn, false>), dim3((unsigned)grid), dim3(256), 0, stream, a);
  }
  return (int)hipGetLastError();
}

}  // namespace

int linear_mfma_max_kp() { return kLmMaxK; }

int launch_linear_mfma(const LinMfmaArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  timing_begin(K_LINEAR_MFMA, stream);
  const int rc = in_dtype == SF_F16    ? launch_lm_d<__half>(a, out_dtype, stream)
                 : in_dtype == SF_BF16 ? launch_lm_d<__hip_bfloat16>(a, out_dtype, stream)
                                       : launch_lm_d<float>(a, out_dtype, stream);
  timing_end(K_LINEAR_MFMA, stream);
  return rc;
}

}  // namespace sf
