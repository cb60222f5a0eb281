// Stage 2 from the prescan bitmap for 3x3 stride-1 convolutions with
// C_in <= 64 (weights resident in LDS) on frames of width 32: row-band
// tiles, lane = output channel.  This is the path of a handed spike map (or
// a separate prescan); with x as input, k_conv_rows_fused runs the same walk
// with the prescan fused in, and the two agree bit for bit.
//
// A block is RB = 4 consecutive output rows of one frame for one group of 64
// output channels; its 16 wavefronts split it into 4 rows x 4 column groups
// of CW = 8 columns.  Wavefront (r, q) owns output row oh0 + r, columns
// 8q .. 8q + 7: lane = output channel, one accumulator register per column.
// Workgroups are persistent over the blocks of the launch; the group's
// weights (row (ci, kh, kw) of 64 channels at 256 B per row) are staged in
// LDS once, with direct global->LDS loads.  Each wavefront reads the channel
// words of its 3 x 10 window positions straight from the bitmap (the next
// block's words are requested before the current block is walked) and walks
// them on the scalar unit (walk_window): a spike (ci, window row ia, window
// column ib) adds weight rows (ci, kh = ia, kw) to accumulators ib - kw,
// fixed registers for compile-time ia, ib; windows whose pixels the prescan
// flagged non-binary multiply by x.  Every output is bias + its taps summed
// in the order (input row, input column, ci).
// (Wider frames keep the pixel-tile kernel: at ResNet50 layer1, 56 wide,
// this formulation measured 263 us against its 117 us -- one LDS round trip
// per spike on each wavefront's critical path, four wavefronts per SIMD.)
// Replaces the reference's sparse_conv3x3s1_nhwc_kernel_8x8/8x16
// (Kernels/conv2d.py:564-724) for these shapes.
#include "sf_tile.h"

namespace sf {

namespace {

constexpr int kBandWaves = 16;

template <int W>
struct BandGeom;
template <>
struct BandGeom<32> {
  static constexpr int Q = 4, RB = 4;
};

template <int W>
struct Band {
  static constexpr int Q = BandGeom<W>::Q, RB = BandGeom<W>::RB;
  static constexpr int CW = W / Q;             // output columns per wavefront
  static constexpr int H = CW + 2;             // window columns per wavefront
  static constexpr int NPOS = (RB + 2) * W;    // window positions of a block
  static constexpr int RUNS = (NPOS + 63) / 64;
  static_assert(Q * RB == kBandWaves && CW * Q == W, "band geometry");
  static_assert(3 * H <= 64, "a wavefront's window words fit one register");
};

// Channel word of window position (row ia, column ib): lane ia * H + ib of
// vw, read on the scalar unit.
template <typename M, int H>
struct LaneWords {
  M vw;
  __device__ __forceinline__ M operator()(int ia, int ib) const {
    const int l = ia * H + ib;
    if constexpr (sizeof(M) == 8) {
      const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)vw, l);
      const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(vw >> 32), l);
      return ((M)hi << 32) | lo;
    } else {
      return __builtin_amdgcn_readlane(vw, l);
    }
  }
};

// x(ci, input row oh - 1 + ia, column c0 - 1 + ib) of the value path; xw =
// element offset of (row oh - 1, column c0 - 1) within a channel plane.
template <typename TIn, int W>
struct WindowValues {
  const TIn* __restrict__ xf;
  int64_t xw;
  int hw;
  __device__ __forceinline__ float operator()(int ci, int ia, int ib) const {
    return to_f32<TIn>(xf[(int64_t)ci * hw + xw + ia * W + ib]);
  }
};

template <typename T>
__device__ __forceinline__ void store2(T* p, float a, float b) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<float2*>(p) = make_float2(a, b);
  } else {
    const T h0 = from_f32<T>(a), h1 = from_f32<T>(b);
    uint16_t u0, u1;
    __builtin_memcpy(&u0, &h0, 2);
    __builtin_memcpy(&u1, &h1, 2);
    *reinterpret_cast<uint32_t*>(p) = (uint32_t)u0 | ((uint32_t)u1 << 16);
  }
}

// The CW outputs of one lane (consecutive columns of one channel row) with
// the widest stores their alignment allows: c0 * sizeof(T) is a multiple of
// CW * sizeof(T), and plane and row strides keep it (W % 4 == 0 or W = 14).
template <typename TOut, int CW>
__device__ __forceinline__ void store_run(TOut* p, const float (&acc)[CW]) {
  if constexpr (CW % 4 == 0) {
#pragma unroll
    for (int k = 0; k < CW; k += 4) store4<TOut>(p + k, acc[k], acc[k + 1], acc[k + 2], acc[k + 3]);
  } else if constexpr (CW % 2 == 0) {
#pragma unroll
    for (int k = 0; k < CW; k += 2) store2<TOut>(p + k, acc[k], acc[k + 1]);
  } else {
#pragma unroll
    for (int k = 0; k < CW; ++k) p[k] = from_f32<TOut>(acc[k]);
  }
}

// Stage the group's weight rows in LDS (row (ci, kh, kw) at 256 B per row):
// direct global->LDS loads (1 KB = four 64-channel rows per instruction)
// when 16-byte pieces of a row are whole (C_out % 4 == 0) -- columns past
// C_out are then zeroed after the first barrier -- else loads through
// registers, zero past C_out.
__device__ __forceinline__ void band_stage_weights(char* smem, const float* __restrict__ wt, int krows, int c_out,
                                                   int co0, int wave, int lane, bool direct) {
  float* wl = reinterpret_cast<float*>(smem);
  if (direct) {
    const int units = (krows + 3) / 4;
    for (int u = wave; u < units; u += kBandWaves) {
      const int row = u * 4 + (lane >> 4);
      const int col = co0 + 4 * (lane & 15);
      const float* src = (row < krows && col < c_out) ? wt + (int64_t)row * c_out + col : wt;
      __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)(smem + u * 1024), 16, 0, 0);
    }
  } else {
    const int nw = krows * 64;
    const bool cok = co0 + lane < c_out;
    const int cc = cok ? co0 + lane : 0;
    for (int i0 = wave * 64 + lane; i0 < nw; i0 += 64 * kBandWaves * 4) {
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + 64 * kBandWaves * u;
        v[u] = wt[(int64_t)((i < nw ? i : 0) >> 6) * c_out + cc];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + 64 * kBandWaves * u;
        if (i < nw) wl[i] = cok ? v[u] : 0.f;
      }
    }
  }
}

// Words of this wavefront's window from the bitmap (lane j < 3 H: window
// row j / H, column j % H; zero outside the frame).
template <typename M, int W>
__device__ __forceinline__ M band_bitmap_words(const M* __restrict__ fb, const ConvArgs& a, int oh, int c0,
                                               int lane) {
  typedef Band<W> B;
  const int ia = lane / B::H, ib = lane - ia * B::H;
  const int ih = oh - 1 + ia, col = c0 - 1 + ib;
  const bool ok = lane < 3 * B::H && ih >= 0 && ih < a.h_in && col >= 0 && col < W;
  return ok ? fb[(int64_t)ih * W + col] : (M)0;
}

// wbytes = weight rows rounded up to whole 1 KB load units.
template <typename TIn, typename TOut, int CWP, int W>
__global__ __launch_bounds__(64 * kBandWaves) void k_conv_band(ConvArgs a, const TIn* __restrict__ x,
                                                               const uint32_t* __restrict__ bits,
                                                               const uint32_t* __restrict__ flags,
                                                               const float* __restrict__ wt,
                                                               const float* __restrict__ bias_p,
                                                               TOut* __restrict__ y, int groups, int krows) {
  typedef Band<W> B;
  typedef typename Word<CWP>::type M;
  extern __shared__ __align__(16) char smem[];
  float* wl = reinterpret_cast<float*>(smem);
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = xcd_local_block((int)blockIdx.x, (int)gridDim.x);
  const int grp = blk % groups;
  const int co0 = grp * 64;
  const bool direct = a.c_out % 4 == 0;
  const int hw = a.hw_in;
  const int bpf = (a.h_out + B::RB - 1) / B::RB;  // blocks per frame
  const int64_t nblocks = a.n * (int64_t)bpf;
  const int64_t bstride = (int64_t)(gridDim.x / groups);
  const int r = wave / B::Q, c0 = (wave % B::Q) * B::CW;
  const char* wlb = smem + lane * 4;
  const float bias = (bias_p != nullptr && co0 + lane < a.c_out) ? bias_p[co0 + lane] : 0.f;
  const M* mbits = reinterpret_cast<const M*>(bits);

  // The weights stream in first; the first block's words follow.
  band_stage_weights(smem, wt, krows, a.c_out, co0, wave, lane, direct);
  int64_t b = blk / groups;
  M nvw = 0;
  bool nvalue = false;
  if (b < nblocks) {
    const int64_t frame = b / bpf;
    const int oh = (int)(b - frame * bpf) * B::RB + r;
    nvw = band_bitmap_words<M, W>(mbits + frame * (int64_t)hw, a, oh, c0, lane);
    nvalue = oh < a.h_out && rows_value_path(a, flags, frame, oh - 1, oh + 1);
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wavefront's direct weight loads have landed
  __syncthreads();
  if (direct && co0 + 64 > a.c_out) {
    for (int i = threadIdx.x; i < krows * 64; i += 64 * kBandWaves)
      if (co0 + (i & 63) >= a.c_out) wl[i] = 0.f;
    __syncthreads();
  }

  for (; b < nblocks; b += bstride) {
    const int64_t frame = b / bpf;
    const int oh = (int)(b - frame * bpf) * B::RB + r;
    const M vw = nvw;
    const bool value = nvalue;
    const int64_t bn = b + bstride;  // the next block of this workgroup
    if (bn < nblocks) {
      const int64_t frame_n = bn / bpf;
      const int ohn = (int)(bn - frame_n * bpf) * B::RB + r;
      nvw = band_bitmap_words<M, W>(mbits + frame_n * (int64_t)hw, a, ohn, c0, lane);
      nvalue = ohn < a.h_out && rows_value_path(a, flags, frame_n, ohn - 1, ohn + 1);
    }
    if (oh < a.h_out) {
      float acc[B::CW];
#pragma unroll
      for (int i = 0; i < B::CW; ++i) acc[i] = bias;
      const LaneWords<M, B::H> words{vw};
      const WindowValues<TIn, W> xval{x + frame * (int64_t)a.c_in * hw, (int64_t)(oh - 1) * W + (c0 - 1), hw};
      const bool row0 = oh >= 1, row2 = oh + 1 < a.h_in;
      if (value) walk_window<0, B::H, 0, B::CW, true, M>(acc, words, wlb, xval, row0, row2);
      else walk_window<0, B::H, 0, B::CW, false, M>(acc, words, wlb, xval, row0, row2);
      if (co0 + lane < a.c_out)
        store_run<TOut, B::CW>(y + ((int64_t)frame * a.c_out + co0 + lane) * a.hw_out + oh * W + c0, acc);
    }
  }
}

size_t band_lds_bytes(int c_in) { return (size_t)((c_in * 9 + 3) / 4) * 1024; }

template <typename TIn, typename TOut, int CWP>
int launch_band_t(const ConvArgs& a, hipStream_t stream) {
  constexpr int W = 32;
  const int groups = (a.c_out + 63) / 64;
  const int krows = a.c_in * 9;
  const int64_t nblocks = a.n * (int64_t)((a.h_out + Band<W>::RB - 1) / Band<W>::RB);
  const int per_group = (int)(nblocks < num_cus() ? nblocks : num_cus());
  const int grid = groups * (per_group > 0 ? per_group : 1);
  constexpr auto kern = k_conv_band<TIn, TOut, CWP, W>;
  const int e = set_lds_limit_once<kern>(kMaxLdsBytes);
  if (e != (int)hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * kBandWaves), band_lds_bytes(a.c_in), stream, a,
                     static_cast<const TIn*>(a.x), a.bits, a.flags, a.wt, a.bias, static_cast<TOut*>(a.y), groups,
                     krows);
  return (int)hipGetLastError();
}

template <typename TIn, typename TOut>
int launch_band_c(const ConvArgs& a, hipStream_t stream) {
  return a.cwp == 2 ? launch_band_t<TIn, TOut, 2>(a, stream) : launch_band_t<TIn, TOut, 1>(a, stream);
}

}  // namespace

bool band_applicable(const ConvArgs& a) {
  return a.k == 3 && a.s == 1 && a.p == 1 && a.c_in <= 64 && a.cwp <= 2 && a.h_out == a.h_in &&
         a.w_out == a.w_in && a.w_in == 32 && a.n * (int64_t)a.h_out < (1ll << 30) &&
         band_lds_bytes(a.c_in) <= (size_t)kMaxLdsBytes;
}

int launch_conv_band(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  timing_begin(K_ROWS, stream);
  int rc;
  if (in_dtype == SF_F32) rc = launch_band_c<float, float>(a, stream);
  else if (in_dtype == SF_F16) rc = out_dtype == SF_F32 ? launch_band_c<__half, float>(a, stream)
                                                        : launch_band_c<__half, __half>(a, stream);
  else rc = out_dtype == SF_F32 ? launch_band_c<__hip_bfloat16, float>(a, stream)
                                : launch_band_c<__hip_bfloat16, __hip_bfloat16>(a, stream);
  timing_end(K_ROWS, stream);
  return rc;
}

}  // namespace sf
