// Stage 1 fused into Stage 2 for 3x3 stride-1 convolutions on 32-wide
// frames with C_in <= 64 (the small-layer case): one launch reads the
// activations, builds the spike bitmap of a block of rows in LDS and
// scatters its spikes.  No bitmap leaves the chip and there is no second
// launch.
//
// Workgroup = RB = 4 consecutive output rows of one frame x one group of 64
// output channels, 16 wavefronts.  Wavefront (r, q) owns output row oh0 + r,
// columns 8q .. 8q + 7 (lane = output channel, one accumulator register per
// column), so a CU runs 16 short spike walks instead of 4 long ones.
//  1. The group's weights (row (ci, kh, kw) of 64 channels at 256 B per
//     row) stream into LDS with direct global->LDS loads; they stay there
//     for every row block the workgroup takes.  The wavefronts read the
//     block's (RB + 2) x 32 halo positions of x: a unit (run of 64 positions
//     = two frame rows, slice of 16 channels) is 16 loads per lane, each a
//     coalesced 256-byte run of one channel.  Bit = |x| >= cutoff, the
//     prescan's rule (k_pack); the unit writes its 16-bit slice of each
//     position's channel word into LDS.  Rows outside the frame get zero
//     words.  The block's non-binary flag is the OR over all its elements.
//  2. After one barrier each wavefront reads the words of its 3 x 10 halo
//     positions into one register (position j in lane j) and walks them on
//     the scalar unit (walk_window): a spike (ci, input row ia, halo column
//     ib) adds weight rows (ci, kh = ia, kw) to accumulators ib - kw, fixed
//     registers for compile-time ia, ib.  Non-binary blocks multiply by x.
//  3. Each lane stores its 8 output columns as two 16-byte runs.
// Every output is bias + its taps summed in the order (input row, input
// column, ci), the order of k_conv_band (the same walk from the bitmap):
// the two kernels agree bit for bit.
// Replaces the reference's prescan + sparse_conv3x3s1_nhwc_kernel_8x8 pair
// (Kernels/conv2d.py:564-643, 986) for these shapes.
#include "sf_tile.h"

namespace sf {

namespace {

constexpr int kFW = 32;               // frame width
constexpr int kFCW = 8;               // output columns per wavefront
constexpr int kFQ = kFW / kFCW;       // column quarters per row
constexpr int kFRB = 4;               // output rows per block
constexpr int kFNW = kFRB * kFQ;      // wavefronts per workgroup
constexpr int kFPos = (kFRB + 2) * kFW;  // halo positions of a block
constexpr int kFHalo = kFCW + 2;      // halo columns of a wavefront

static_assert(kFPos % 64 == 0, "halo positions come in runs of 64");
static_assert(3 * kFHalo <= 64, "a wavefront's halo words fit one register");

// Channel word of halo position (input row ia, halo column ib): lane
// ia * kFHalo + ib of vw, read on the scalar unit.
template <typename M>
struct HaloWords {
  M vw;
  __device__ __forceinline__ M operator()(int ia, int ib) const {
    const int l = ia * kFHalo + ib;
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
template <typename TIn>
struct HaloValues {
  const TIn* __restrict__ xf;
  int64_t xw;
  int hw;
  __device__ __forceinline__ float operator()(int ci, int ia, int ib) const {
    return to_f32<TIn>(xf[(int64_t)ci * hw + xw + ia * kFW + ib]);
  }
};

// wbytes = weight rows rounded up to whole 1 KB load units; the block's
// channel words (CWP 32-bit words per position, as 16-bit slices) and the
// per-wavefront non-binary flags follow.
template <typename TIn, typename TOut, int CWP>
__global__ __launch_bounds__(64 * kFNW) void k_conv_rows_fused(ConvArgs a, const TIn* __restrict__ x,
                                                               const float* __restrict__ wt,
                                                               const float* __restrict__ bias_p,
                                                               TOut* __restrict__ y, int groups, int krows,
                                                               int wbytes, float cut) {
  typedef typename Word<CWP>::type M;
  constexpr int SL = 2 * CWP;  // 16-bit slices per position word
  extern __shared__ __align__(16) char smem[];
  uint16_t* s_slice = reinterpret_cast<uint16_t*>(smem + wbytes);
  const M* s_words = reinterpret_cast<const M*>(smem + wbytes);
  uint32_t* s_nb = reinterpret_cast<uint32_t*>(smem + wbytes + kFPos * SL * 2);
  float* wl = reinterpret_cast<float*>(smem);
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = xcd_local_block((int)blockIdx.x, (int)gridDim.x);
  const int grp = blk % groups;
  const int co0 = grp * 64;
  const bool direct = a.c_out % 4 == 0;

  // Weights: direct loads (1 KB = four 64-channel rows per instruction) when
  // 16-byte pieces of a row are whole (C_out % 4 == 0); columns past C_out
  // are zeroed after the first barrier.  Otherwise loads through registers,
  // zero past C_out.
  if (direct) {
    const int units = (krows + 3) / 4;
    for (int u = wave; u < units; u += kFNW) {
      const int row = u * 4 + (lane >> 4);
      const int col = co0 + 4 * (lane & 15);
      const float* src = (row < krows && col < a.c_out) ? wt + (int64_t)row * a.c_out + col : wt;
      __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)(smem + u * 1024), 16, 0, 0);
    }
  } else {
    const int nw = krows * 64;
    const bool cok = co0 + lane < a.c_out;
    const int cc = cok ? co0 + lane : 0;
    for (int i0 = threadIdx.x; i0 < nw; i0 += 64 * kFNW * 4) {
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + 64 * kFNW * u;
        v[u] = wt[(int64_t)((i < nw ? i : 0) >> 6) * a.c_out + cc];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + 64 * kFNW * u;
        if (i < nw) wl[i] = cok ? v[u] : 0.f;
      }
    }
  }

  const float bias = (bias_p != nullptr && co0 + lane < a.c_out) ? bias_p[co0 + lane] : 0.f;
  const int bpf = (a.h_out + kFRB - 1) / kFRB;  // row blocks per frame
  const int64_t nblocks = a.n * (int64_t)bpf;
  const int64_t bstride = (int64_t)(gridDim.x / groups);
  const int r = wave / kFQ, c0 = (wave % kFQ) * kFCW;
  const int hw = a.hw_in;
  const char* wlb = smem + lane * 4;
  bool first = true;
  for (int64_t b = blk / groups; b < nblocks; b += bstride) {
    const int64_t frame = b / bpf;
    const int oh0 = (int)(b - frame * bpf) * kFRB;
    const TIn* __restrict__ xf = x + frame * (int64_t)a.c_in * hw;
    // The previous block's words and flags have been read by every wavefront.
    if (!first) __syncthreads();

    // 1. x -> channel words of the block's halo positions.
    uint32_t nb = 0u;
    for (int u = wave; u < 3 * SL; u += kFNW) {
      const int pb = u / SL, cs = u - pb * SL;
      const int p = pb * 64 + lane;
      const int ih = oh0 - 1 + p / kFW;
      const bool ok = ih >= 0 && ih < a.h_in;
      const int64_t off = ok ? (int64_t)(cs * 16) * hw + ih * kFW + (p % kFW) : 0;
      float v[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = (ok && cs * 16 + j < a.c_in) ? to_f32<TIn>(xf[off + (int64_t)j * hw]) : 0.f;
      uint32_t piece = 0u;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        piece |= (fabsf(v[j]) >= cut ? 1u : 0u) << j;
        nb |= (v[j] != 0.f && v[j] != 1.f) ? 1u : 0u;
      }
      s_slice[p * SL + cs] = (uint16_t)piece;
    }
    const uint64_t nb_any = __ballot(nb != 0u);
    if (lane == 0) s_nb[wave] = nb_any != 0ull ? 1u : 0u;
    if (first) __builtin_amdgcn_s_waitcnt(0);  // this wavefront's direct weight loads have landed
    __syncthreads();
    if (first && direct && co0 + 64 > a.c_out) {
      for (int i = threadIdx.x; i < krows * 64; i += 64 * kFNW)
        if (co0 + (i & 63) >= a.c_out) wl[i] = 0.f;
      __syncthreads();
    }
    first = false;

    // 2. Walk this wavefront's halo words.
    const bool value = __ballot(lane < kFNW && s_nb[lane < kFNW ? lane : 0] != 0u) != 0ull;
    const int oh = oh0 + r;
    if (oh < a.h_out) {
      M vw = 0;
      {
        const int ia = lane / kFHalo, ib = lane - ia * kFHalo;
        const int col = c0 - 1 + ib;
        if (lane < 3 * kFHalo && col >= 0 && col < kFW) vw = s_words[(r + ia) * kFW + col];
      }
      float acc[kFCW];
#pragma unroll
      for (int i = 0; i < kFCW; ++i) acc[i] = bias;
      const HaloWords<M> words{vw};
      const HaloValues<TIn> xval{xf, (int64_t)(oh - 1) * kFW + (c0 - 1), hw};
      // Rows outside the frame have zero words.
      if (value) walk_window<0, kFHalo, 0, kFCW, true, M>(acc, words, wlb, xval, true, true);
      else walk_window<0, kFHalo, 0, kFCW, false, M>(acc, words, wlb, xval, true, true);

      // 3. Store.
      if (co0 + lane < a.c_out) {
        TOut* yr = y + ((int64_t)frame * a.c_out + co0 + lane) * a.hw_out + oh * kFW + c0;
#pragma unroll
        for (int k = 0; k < kFCW; k += 4) store4<TOut>(yr + k, acc[k], acc[k + 1], acc[k + 2], acc[k + 3]);
      }
    }
  }
}

template <typename TIn, typename TOut, int CWP>
int launch_fused_t(const ConvArgs& a, float cut, hipStream_t stream) {
  const int groups = (a.c_out + 63) / 64;
  const int krows = a.c_in * 9;
  const int wbytes = ((krows + 3) / 4) * 1024;
  const size_t lds = (size_t)wbytes + (size_t)kFPos * 2 * CWP * 2 + kFNW * 4;
  const int64_t nblocks = a.n * (int64_t)((a.h_out + kFRB - 1) / kFRB);
  const int per_group = (int)(nblocks < num_cus() ? nblocks : num_cus());
  const int grid = groups * (per_group > 0 ? per_group : 1);
  constexpr auto kern = k_conv_rows_fused<TIn, TOut, CWP>;
  const int e = set_lds_limit_once<kern>(kMaxLdsBytes);
  if (e != (int)hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * kFNW), lds, stream, a, static_cast<const TIn*>(a.x), a.wt, a.bias,
                     static_cast<TOut*>(a.y), groups, krows, wbytes, cut);
  return (int)hipGetLastError();
}

template <typename TIn, typename TOut>
int launch_fused_d(const ConvArgs& a, float cut, hipStream_t stream) {
  return a.cwp == 1 ? launch_fused_t<TIn, TOut, 1>(a, cut, stream) : launch_fused_t<TIn, TOut, 2>(a, cut, stream);
}

}  // namespace

bool rows_fused_applicable(const ConvArgs& a) {
  const int64_t wbytes = (int64_t)((a.c_in * 9 + 3) / 4) * 1024;
  return a.k == 3 && a.s == 1 && a.p == 1 && a.c_in <= 64 && a.cwp <= 2 && a.h_out == a.h_in &&
         a.w_out == a.w_in && a.w_in == kFW && a.n * (int64_t)a.h_out < (1ll << 30) &&
         (int64_t)a.c_in * a.hw_in < (1ll << 31) &&
         wbytes + (int64_t)kFPos * 2 * a.cwp * 2 + kFNW * 4 <= kMaxLdsBytes;
}

int launch_conv_rows_fused(const ConvArgs& a, int in_dtype, int out_dtype, float cutoff, hipStream_t stream) {
  timing_begin(K_ROWS_FUSED, stream);
  int rc;
  if (in_dtype == SF_F32) rc = launch_fused_d<float, float>(a, cutoff, stream);
  else if (in_dtype == SF_F16) rc = out_dtype == SF_F32 ? launch_fused_d<__half, float>(a, cutoff, stream)
                                                        : launch_fused_d<__half, __half>(a, cutoff, stream);
  else rc = out_dtype == SF_F32 ? launch_fused_d<__hip_bfloat16, float>(a, cutoff, stream)
                                : launch_fused_d<__hip_bfloat16, __hip_bfloat16>(a, cutoff, stream);
  timing_end(K_ROWS_FUSED, stream);
  return rc;
}

}  // namespace sf
