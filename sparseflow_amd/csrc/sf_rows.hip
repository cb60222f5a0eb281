// Stage 2, row-tile scatter formulation: 3x3 stride-1 convolutions whose
// weights for 64 output channels fit in LDS (C_in <= 64) on frames of width
// 32 (the small-frame case, where one 64-pixel pixel tile per wavefront would
// leave most of the chip idle).
//
// One wavefront owns one output row of one frame for 64 output channels
// (lane = output channel, one accumulator register per output pixel).  The
// weights of the workgroup's 64-channel group stay in LDS for the whole
// (persistent) launch.  The wavefront walks the spike bitmap of the three
// input rows on the scalar unit (walk_window): every active (ci, ih, iw)
// contributes weight rows (ci, kh = ih - oh + 1, kw) to output columns
// iw + 1 - kw, and because the input position is a compile-time loop index,
// every target accumulator is a fixed register.  Each weight row is read
// from LDS at an immediate offset.  The finished row is transposed in registers (DPP row shifts and
// quad permutes) so that each store instruction writes whole frame rows of
// 64/QP channels as float4 runs.
//
// Output element (co, oh, ow) = bias[co] + its taps summed by one lane in the
// order (input row, input column, ci): deterministic from run to run.
// Replaces the reference's sparse_conv3x3s1_nhwc_kernel_8x8/8x16
// (Kernels/conv2d.py:564-724) for these shapes.
#include "sf_tile.h"

namespace sf {

namespace {


// Word of halo position p (lane p & 63 of v0 for p < 64, else of v1) on the
// scalar unit; p is a compile-time constant once the walks are unrolled.
template <typename M>
__device__ __forceinline__ M rl_word(M v0, M v1, int p) {
  const M v = p < 64 ? v0 : v1;
  if constexpr (sizeof(M) == 8) {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, p & 63);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), p & 63);
    return ((M)hi << 32) | lo;
  } else {
    return __builtin_amdgcn_readlane(v, p & 63);
  }
}

// Channel word of window position (input row oh - 1 + ia, column ib): lane
// p & 63 of v0 (p < 64) or v1, p = ia * W + ib, read on the scalar unit.
template <int W, typename M>
struct RowWords {
  M v0, v1;
  __device__ __forceinline__ M operator()(int ia, int ib) const { return rl_word<M>(v0, v1, ia * W + ib); }
};

// x(ci, input row oh - 1 + ia, column ib) of the value path; xr = element
// offset of row oh - 1 within a channel plane.
template <int W, typename TIn>
struct RowValues {
  const TIn* __restrict__ xf;
  int64_t xr;
  int hw;
  __device__ __forceinline__ float operator()(int ci, int ia, int ib) const {
    return to_f32<TIn>(xf[(int64_t)ci * hw + xr + ia * W + ib]);
  }
};

template <int W, int QP, int CWP, bool VALUE, typename TIn>
__device__ __forceinline__ void scatter_tile(float (&acc)[4 * QP], const ConvArgs& a,
                                             const typename Word<CWP>::type* __restrict__ bits,
                                             const TIn* __restrict__ x, int64_t frame, int oh, const char* wlb) {
  typedef typename Word<CWP>::type M;
  const M* __restrict__ fb = bits + frame * (int64_t)a.hw_in;
  const TIn* __restrict__ xf = x + frame * (int64_t)a.c_in * a.hw_in;
  // Words of the 3 x W window positions (rows oh-1 .. oh+1), position p in
  // lane p & 63 of v0 / v1: two vector loads instead of batches of dependent
  // scalar loads; rows outside the frame read as zero words.
  const int lane = lane_id();
  M v0 = 0, v1 = 0;
  {
    const int p0 = lane, p1 = 64 + lane;
    const int ih0 = oh - 1 + p0 / W, ih1 = oh - 1 + p1 / W;
    if (p0 < 3 * W && ih0 >= 0 && ih0 < a.h_in) v0 = fb[(int64_t)(oh - 1) * W + p0];
    if (p1 < 3 * W && ih1 >= 0 && ih1 < a.h_in) v1 = fb[(int64_t)(oh - 1) * W + p1];
  }
  walk_window<0, W, 1, 4 * QP, VALUE, M>(acc, RowWords<W, M>{v0, v1}, wlb,
                                          RowValues<W, TIn>{xf, (int64_t)(oh - 1) * W, a.hw_in}, oh >= 1,
                                          oh + 1 < a.h_in);
}

// OR of the non-binary chunk flags covering input rows oh-1 .. oh+1.
__device__ __forceinline__ bool rows_value_path(const ConvArgs& a, const uint32_t* __restrict__ flags, int64_t frame,
                                                int oh) {
  const int ih_a = max(0, oh - 1), ih_b = min(a.h_in - 1, oh + 1);
  const int64_t c_a = ((int64_t)ih_a * a.w_in) / a.chunk;
  const int64_t c_b = ((int64_t)ih_b * a.w_in + a.w_in - 1) / a.chunk;
  const uint32_t* __restrict__ fl = flags + frame * a.chunks_per_frame;
  uint32_t f = 0u;
  for (int64_t q = c_a; q <= c_b; ++q) f |= fl[q];
  return f != 0u;
}

// The bitmap, flags, x and weights are passed as separate restrict-qualified
// arguments so that their uniform loads compile to scalar (SMEM) loads.
// NWR wavefronts per workgroup: 16, or 4 when 16-wave workgroups would leave
// CUs idle (few rows: the weights are then loaded by more workgroups).
template <typename TIn, typename TOut, int W, int CWP, int NWR>
__global__ __launch_bounds__(64 * NWR) void k_conv_rows(ConvArgs a, const uint32_t* __restrict__ bits,
                                                               const uint32_t* __restrict__ flags,
                                                               const TIn* __restrict__ x, const float* __restrict__ wt,
                                                               const float* __restrict__ bias_p, TOut* __restrict__ y,
                                                               int groups, int krows) {
  typedef typename Word<CWP>::type M;
  constexpr int QP = W <= 32 ? 8 : 16;  // quad slots per row (power of two >= W/4)
  extern __shared__ __align__(16) char smem[];
  float* wl = reinterpret_cast<float*>(smem);
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = blockIdx.x % groups;
  const int co0 = grp * 64;
  // Weights straight from global memory into LDS (direct loads, 1 KB = four
  // 64-channel rows per wavefront instruction, all in flight; 16-byte pieces
  // of a row need C_out % 4 == 0); columns past C_out are then zeroed.
  // Otherwise eight loads in flight per thread through registers.
  if (a.c_out % 4 != 0) {
    const int nw = krows * 64;
    const int c = threadIdx.x & 63;  // the stride is a multiple of 64
    const bool cok = co0 + c < a.c_out;
    const int cc = cok ? co0 + c : 0;
    for (int i0 = threadIdx.x; i0 < nw; i0 += 64 * NWR * 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = i0 + 64 * NWR * u;
        const int r = (i < nw ? i : 0) >> 6;
        v[u] = wt[(int64_t)r * a.c_out + cc];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = i0 + 64 * NWR * u;
        if (i < nw) wl[i] = cok ? v[u] : 0.f;
      }
    }
  } else {
    const int units = (krows + 3) / 4;
    for (int u = wave; u < units; u += NWR) {
      const int r = u * 4 + (lane >> 4);
      const int col = co0 + 4 * (lane & 15);
      const float* src = (r < krows && col < a.c_out) ? wt + (int64_t)r * a.c_out + col : wt;
      __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)(smem + u * 1024), 16, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);
    if (co0 + 64 > a.c_out) {
      __syncthreads();
      for (int i = threadIdx.x; i < krows * 64; i += 64 * NWR)
        if (co0 + (i & 63) >= a.c_out) wl[i] = 0.f;
    }
  }
  __syncthreads();
  const char* wlb = smem + lane * 4;
  const float bias = (bias_p != nullptr && co0 + lane < a.c_out) ? bias_p[co0 + lane] : 0.f;
  const int rows_total = (int)(a.n * a.h_out);
  const int wpg = (int)(gridDim.x / groups) * NWR;
  const int q = lane & (QP - 1);
  const int cbase = lane & ~(QP - 1);
  for (int t = (int)(blockIdx.x / groups) * NWR + wave; t < rows_total; t += wpg) {
    const int frame = t / a.h_out;
    const int oh = t - frame * a.h_out;
    float acc[4 * QP];
#pragma unroll
    for (int i = 0; i < 4 * QP; ++i) acc[i] = i < W ? bias : 0.f;
    const M* mbits = reinterpret_cast<const M*>(bits);
    if (rows_value_path(a, flags, frame, oh)) scatter_tile<W, QP, CWP, true, TIn>(acc, a, mbits, x, frame, oh, wlb);
    else scatter_tile<W, QP, CWP, false, TIn>(acc, a, mbits, x, frame, oh, wlb);
    butterfly<1, QP>(acc, lane);
    butterfly<2, QP>(acc, lane);
    butterfly<4, QP>(acc, lane);
    if constexpr (QP == 16) butterfly<8, QP>(acc, lane);
    // Slot k of lane L now holds output channel (L & ~(QP-1)) | k, columns 4*(L & (QP-1)) .. +3.
    if (4 * q < W) {
      TOut* yr = y + ((int64_t)frame * a.c_out + co0 + cbase) * a.hw_out + oh * W + 4 * q;
#pragma unroll
      for (int k = 0; k < QP; ++k) {
        if (co0 + cbase + k < a.c_out)
          store4<TOut>(yr + (int64_t)k * a.hw_out, acc[4 * k], acc[4 * k + 1], acc[4 * k + 2], acc[4 * k + 3]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// K-chunked variant for layers whose weights do not fit LDS (C_in > 64).
//
// Tile = TH full rows of a W-wide frame (TH*W <= 64 output pixels, contiguous
// in the output plane), lane = output channel.  Weights are consumed in
// chunks of one 32-channel bitmap word (32 ci x 9 taps x 64 co = 72 KB),
// double-buffered in LDS: while the workgroup's 16 wavefronts walk chunk c
// from one buffer, chunk c+1 streams into the other with direct global->LDS
// loads.  One barrier per chunk.  With at most two chunks both stay resident
// and the wavefronts never synchronise.
// ---------------------------------------------------------------------------

constexpr int kChunkBytes = 32 * 9 * 64 * 4;  // one chunk of weights: 72 KB = 72 units of 1 KB

// Issue the direct-to-LDS loads of weight chunk c into `buf`.  Each 1 KB unit
// (4 weight rows x 64 channels) is one wavefront instruction: lane l carries
// row 4u + l/16, channels 4*(l%16) .. +3.  Rows past C_in and channels past
// C_out read a valid but unrelated address; those values are never used.
__device__ __forceinline__ void load_chunk(char* buf, const float* __restrict__ wt, int c, int krows, int c_out,
                                           int co0, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < (kChunkBytes / 1024 + kRowsWaves - 1) / kRowsWaves; ++j) {
    const int u = wave + kRowsWaves * j;
    if (u < kChunkBytes / 1024) {
      const int row = c * (32 * 9) + u * 4 + (lane >> 4);
      const int col = co0 + 4 * (lane & 15);
      const float* src = (row < krows && col < c_out) ? wt + (int64_t)row * c_out + col : wt;
      __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)(buf + u * 1024), 16, 0, 0);
    }
  }
}

struct KcTile {
  // The chunk's bitmap words of the (TH + 2) x W halo positions, position p
  // in lane p & 63 of vw0 (p < 64) or vw1: fetched with two vector loads and
  // read on the scalar unit with readlane at compile-time lanes.
  uint32_t vw0, vw1;
  const void* x;            // x plane of the frame (value path)
  int64_t xrow;             // element offset of input row oh0 - 1 within a channel plane
  const char* wlb;          // LDS weight chunk + lane offset
  int oh0, h, cwp, hw, in_dtype, c0;  // c0 = first channel of the chunk
  bool value;               // tile reads non-binary inputs: multiply by x
};

// Spikes of halo position (IA, IB) (input row oh0-1+IA, column IB) whose
// chunk word is m.  Every weight row lands in a compile-time accumulator;
// binary tiles multiply by exactly 1.
template <int TH, int W, int IA, int IB>
__device__ __forceinline__ void kc_position(float (&acc)[64], uint32_t m, const KcTile& k) {
  while (m) {
    const int bit = __builtin_ctz(m);
    m &= m - 1;
    float xv = 1.f;
    if (k.value) xv = load_x(k.x, k.in_dtype, (int64_t)(k.c0 + bit) * k.hw + k.xrow + IA * W + IB);
    const char* base = k.wlb + bit * (9 * 256);
#pragma unroll
    for (int kh = 0; kh < 3; ++kh) {
      const int r = IA - kh;
      if (r < 0 || r >= TH) continue;
#pragma unroll
      for (int kw = 0; kw < 3; ++kw) {
        const int xo = IB + 1 - kw;
        if (xo < 0 || xo >= W) continue;
        acc[r * W + xo] = fmaf(xv, *reinterpret_cast<const float*>(base + (kh * 3 + kw) * 256), acc[r * W + xo]);
      }
    }
  }
}

template <int TH, int W, int IA, int B0, int U, int NB>
__device__ __forceinline__ void kc_batch_walk(float (&acc)[64], const uint32_t (&mw)[8], const KcTile& k) {
  if constexpr (U < NB) {
    kc_position<TH, W, IA, B0 + U>(acc, mw[U], k);
    kc_batch_walk<TH, W, IA, B0, U + 1, NB>(acc, mw, k);
  }
}

template <int P>
__device__ __forceinline__ uint32_t kc_word(const KcTile& k) {
  static_assert(P < 128, "halo positions fit two words per lane");
  return __builtin_amdgcn_readlane(P < 64 ? k.vw0 : k.vw1, P & 63);
}

template <int P, int U, int NB>
__device__ __forceinline__ void kc_fill(uint32_t (&mw)[8], const KcTile& k) {
  if constexpr (U < NB) {
    mw[U] = kc_word<P + U>(k);
    kc_fill<P, U + 1, NB>(mw, k);
  }
}

template <int TH, int W, int IA, int B0>
__device__ __forceinline__ void kc_row(float (&acc)[64], const KcTile& k) {
  if constexpr (B0 < W) {
    constexpr int NB = (W - B0) < 8 ? (W - B0) : 8;
    uint32_t mw[8];
    kc_fill<IA * W + B0, 0, NB>(mw, k);
    kc_batch_walk<TH, W, IA, B0, 0, NB>(acc, mw, k);
    kc_row<TH, W, IA, B0 + 8>(acc, k);
  }
}

template <int TH, int W, int IA>
__device__ __forceinline__ void kc_rows(float (&acc)[64], const KcTile& k) {
  if constexpr (IA < TH + 2) {
    const int ih = k.oh0 - 1 + IA;
    if (ih >= 0 && ih < k.h) kc_row<TH, W, IA, 0>(acc, k);
    kc_rows<TH, W, IA + 1>(acc, k);
  }
}

// Chunk c's words of the tile's halo positions (rows oh0 - 1 .. oh0 + TH of
// the frame; rows outside it read position 0 and are never walked).
template <int TH, int W>
__device__ __forceinline__ void kc_load_words(uint32_t& v0, uint32_t& v1, const uint32_t* __restrict__ fbits,
                                              int oh0, int h, int cwp, int lane, int c) {
  constexpr int NP = (TH + 2) * W;
  const int p0 = lane, p1 = 64 + lane;
  const int ih0 = oh0 - 1 + p0 / W, ih1 = oh0 - 1 + p1 / W;
  const bool ok0 = p0 < NP && ih0 >= 0 && ih0 < h, ok1 = p1 < NP && ih1 >= 0 && ih1 < h;
  const int64_t q0 = ok0 ? (int64_t)(oh0 - 1) * W + p0 : 0, q1 = ok1 ? (int64_t)(oh0 - 1) * W + p1 : 0;
  v0 = fbits[q0 * cwp + c];
  v1 = fbits[q1 * cwp + c];
}

template <int TH, int W>
__global__ __launch_bounds__(64 * kRowsWaves) void k_conv_rows_kc(ConvArgs a, const uint32_t* __restrict__ bits,
                                                                  const uint32_t* __restrict__ flags,
                                                                  const void* __restrict__ x,
                                                                  const float* __restrict__ wt,
                                                                  const float* __restrict__ bias_p,
                                                                  void* __restrict__ y, int groups, int nchunks,
                                                                  int in_dtype, int out_dtype) {
  // Launched only for planes with h*w % 4 == 0, so every tile's run (TH*W, or
  // an even number of 14-wide rows for the last tile) is whole quads.
  static_assert(TH * W <= 64 && (TH * W) % 4 == 0, "tile must be a whole number of quads within 64 pixels");
  extern __shared__ __align__(16) char smem[];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = blockIdx.x % groups;
  const int co0 = grp * 64;
  const int krows = a.c_in * 9;
  const float bias = (bias_p != nullptr && co0 + lane < a.c_out) ? bias_p[co0 + lane] : 0.f;
  const int h = a.h_in;
  const int tpf = (h + TH - 1) / TH;
  const int total = (int)a.n * tpf;
  const int nblk = (int)(gridDim.x / groups);
  const bool resident = nchunks <= 2;
  const int in_size = in_dtype == SF_F32 ? 4 : 2;

  if (resident) {
    for (int c = 0; c < nchunks; ++c) load_chunk(smem + c * kChunkBytes, wt, c, krows, a.c_out, co0, wave, lane);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  // Passes of kRowsWaves tiles.  With more than two chunks every wavefront
  // takes part in every barrier, including those of a pass past the end.
  for (int pass = (int)(blockIdx.x / groups); pass * kRowsWaves < total; pass += nblk) {
    const int t = pass * kRowsWaves + wave;
    const bool valid = t < total;
    const int frame = valid ? t / tpf : 0;
    const int oh0 = valid ? (t - frame * tpf) * TH : 0;
    float acc[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) acc[i] = i < TH * W ? bias : 0.f;
    KcTile k;
    k.oh0 = oh0;
    k.h = h;
    k.cwp = a.cwp;
    k.hw = a.hw_in;
    k.in_dtype = in_dtype;
    k.x = static_cast<const char*>(x) + (int64_t)frame * a.c_in * a.hw_in * in_size;
    k.xrow = (int64_t)(oh0 - 1) * W;
    k.value = valid && rows_value_path(a, flags, frame, oh0 - 1, oh0 + TH);
    // Chunk 0's halo words; chunk c+1's are requested while chunk c is walked.
    const uint32_t* __restrict__ fbits = bits + (int64_t)frame * a.hw_in * a.cwp;
    uint32_t nw0 = 0u, nw1 = 0u;
    if (valid) kc_load_words<TH, W>(nw0, nw1, fbits, oh0, h, a.cwp, lane, 0);
    if (!resident) {
      __syncthreads();  // the previous pass is done with both buffers
      load_chunk(smem, wt, 0, krows, a.c_out, co0, wave, lane);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
    for (int c = 0; c < nchunks; ++c) {
      // Stream chunk c+1 into the other buffer; it was last read during
      // chunk c-1, which every wavefront finished before the last barrier.
      if (!resident && c + 1 < nchunks)
        load_chunk(smem + ((c + 1) & 1) * kChunkBytes, wt, c + 1, krows, a.c_out, co0, wave, lane);
      if (valid) {
        k.vw0 = nw0;
        k.vw1 = nw1;
        if (c + 1 < nchunks) kc_load_words<TH, W>(nw0, nw1, fbits, oh0, h, a.cwp, lane, c + 1);
        k.c0 = c * 32;
        k.wlb = smem + (c & 1) * kChunkBytes + lane * 4;
        kc_rows<TH, W, 0>(acc, k);
      }
      if (!resident) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
      }
    }
    if (valid) {
      const int npx = min(TH, h - oh0) * W;
      butterfly<1, 16>(acc, lane);
      butterfly<2, 16>(acc, lane);
      butterfly<4, 16>(acc, lane);
      butterfly<8, 16>(acc, lane);
      if (out_dtype == SF_F16) tile_store<__half>(acc, y, a, frame, co0, oh0 * W, npx, lane);
      else if (out_dtype == SF_BF16) tile_store<__hip_bfloat16>(acc, y, a, frame, co0, oh0 * W, npx, lane);
      else tile_store<float>(acc, y, a, frame, co0, oh0 * W, npx, lane);
    }
  }
}

template <int TH, int W>
int launch_kc_t(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  const int groups = (a.c_out + 63) / 64;
  const int nchunks = (a.c_in + 31) / 32;
  const size_t lds = (size_t)2 * kChunkBytes;
  const int64_t tiles = a.n * (int64_t)((a.h_out + TH - 1) / TH);
  const int64_t need = (tiles + kRowsWaves - 1) / kRowsWaves;
  const int per_group = (int)(need < num_cus() ? need : num_cus());
  const int grid = groups * (per_group > 0 ? per_group : 1);
  constexpr auto kern = k_conv_rows_kc<TH, W>;
  const int e = set_lds_limit_once<kern>(kMaxLdsBytes);
  if (e != (int)hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * kRowsWaves), lds, stream, a, a.bits, a.flags, a.x, a.wt, a.bias,
                     a.y, groups, nchunks, in_dtype, out_dtype);
  return (int)hipGetLastError();
}

template <typename TIn, typename TOut, int W, int CWP, int NWR>
int launch_rows_t(const ConvArgs& a, hipStream_t stream) {
  const int groups = (a.c_out + 63) / 64;
  const int krows = a.c_in * 9;
  const size_t lds = (size_t)((krows + 3) / 4) * 1024;  // whole 1 KB load units
  const int64_t rows_total = a.n * (int64_t)a.h_out;
  const int64_t need = (rows_total + NWR - 1) / NWR;
  const int per_group = (int)(need < num_cus() ? need : num_cus());
  const int grid = groups * (per_group > 0 ? per_group : 1);
  constexpr auto kern = k_conv_rows<TIn, TOut, W, CWP, NWR>;
  const int e = set_lds_limit_once<kern>(kMaxLdsBytes);
  if (e != (int)hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * NWR), lds, stream, a, a.bits, a.flags,
                     static_cast<const TIn*>(a.x), a.wt, a.bias, static_cast<TOut*>(a.y), groups, krows);
  return (int)hipGetLastError();
}

template <typename TIn, typename TOut>
int launch_rows_d(const ConvArgs& a, hipStream_t stream) {
  const int groups = (a.c_out + 63) / 64;
  const bool few = a.n * (int64_t)a.h_out * groups < (int64_t)kRowsWaves * num_cus();
  if (few) return a.cwp == 1 ? launch_rows_t<TIn, TOut, 32, 1, 4>(a, stream) : launch_rows_t<TIn, TOut, 32, 2, 4>(a, stream);
  return a.cwp == 1 ? launch_rows_t<TIn, TOut, 32, 1, kRowsWaves>(a, stream)
                    : launch_rows_t<TIn, TOut, 32, 2, kRowsWaves>(a, stream);
}

}  // namespace

namespace {
int g_num_cus[64] = {0};
}  // namespace

int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (g_num_cus[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    g_num_cus[dev] = v;
  }
  return g_num_cus[dev];
}

bool rows_applicable(const ConvArgs& a) {
  return a.k == 3 && a.s == 1 && a.p == 1 && a.c_in <= 64 && a.cwp <= 2 && a.h_out == a.h_in &&
         a.w_out == a.w_in && a.w_out == 32 && a.n * (int64_t)a.h_out < (1ll << 30) &&
         (int64_t)a.c_in * 9 * 64 * 4 <= kMaxLdsBytes;
}

bool rows_kc_applicable(const ConvArgs& a) {
  return a.k == 3 && a.s == 1 && a.p == 1 && a.h_out == a.h_in && a.w_out == a.w_in &&
         (a.w_out == 28 || a.w_out == 14) && a.c_out % 4 == 0 && a.hw_out % 4 == 0 &&
         a.n * (int64_t)a.h_out < (1ll << 30);
}

int launch_conv_rows_kc(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  timing_begin(K_ROWS_KC, stream);
  const int rc = a.w_out == 28 ? launch_kc_t<2, 28>(a, in_dtype, out_dtype, stream)
                               : launch_kc_t<4, 14>(a, in_dtype, out_dtype, stream);
  timing_end(K_ROWS_KC, stream);
  return rc;
}

int launch_conv_rows(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  timing_begin(K_ROWS, stream);
  int rc;
  if (in_dtype == SF_F32) rc = launch_rows_d<float, float>(a, stream);
  else if (in_dtype == SF_F16) rc = out_dtype == SF_F32 ? launch_rows_d<__half, float>(a, stream)
                                                        : launch_rows_d<__half, __half>(a, stream);
  else rc = out_dtype == SF_F32 ? launch_rows_d<__hip_bfloat16, float>(a, stream)
                                : launch_rows_d<__hip_bfloat16, __hip_bfloat16>(a, stream);
  timing_end(K_ROWS, stream);
  return rc;
}

}  // namespace sf
