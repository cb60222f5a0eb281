// Stage 2 on the matrix cores for 3x3 convolutions whose whole reduction is
// one small dense tile: K = C_in * 9 <= 32 (C_in <= 3, the image stem of a
// spiking network).  Every output needs at most 32 MACs, so there is nothing
// worth skipping and the time is the output write; the spike walk, built for
// long sparse reductions, spends several times that on these layers (dense,
// non-binary input: every tap active, value path).
//
// Implicit GEMM: y[p, co] = bias[co] + sum_k A[p, k] W[k, co] with
// A[p, k] = x at tap k of output pixel p where the input's bitmap bit is set
// (the prescan's activity test, so sub-threshold inputs count as zero as on
// every other path), 0 outside the frame.  fp32 matrix cores
// (V_MFMA_F32_16X16X4_F32): exact fp32 products, fp32 sums, no operand split.
//
// A workgroup (4 wavefronts) owns 256 consecutive output pixels of one frame
// for one 64-channel group.  It first stages, with coalesced loads that are
// all in flight together, (i) the input rows those pixels read, masked by the
// bitmap and surrounded by a zero halo, so that A is an LDS read with no
// bounds tests, and (ii) the group's 32 x 64 weight slice.  One wavefront =
// 64 pixels x 64 channels = 4 x 4 MFMA blocks of 16 x 16 (64 accumulators
// per lane), K in steps of 4: lane l holds A[p][k] for pixel l % 16 of a
// pixel block and k = 4 step + l / 16, and B[k][co] for channel l % 16 of a
// channel block.  Accumulator r of block (pb, cb) in lane l is pixel
// 16 pb + 4 (l/16) + r, channel 16 cb + l % 16; the tile leaves through the
// wavefront's LDS region, 16 channels at a time ([16 channels][64 pixels],
// rows padded to 272 bytes: the write and the read-back touch 16 different
// bank groups per 16 lanes), so that each store writes four channel planes x
// 256 contiguous bytes.
//
// Deterministic: each output is one fixed sequence of MFMA accumulations.
// Replaces the reference's dense ALL_ONES tile branch (tl.dot over a tile's
// full K, Kernels/conv2d.py:606-620) for these shapes.
#include "sf_tile.h"

namespace sf {

namespace {

typedef float mc_f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMcWaves = 4;                 // wavefronts per workgroup (one per SIMD)
constexpr int kMcPixels = 64 * kMcWaves;    // output pixels per workgroup
constexpr int kMcSteps = 8;                 // K steps of 4: K <= 32
constexpr int kMcMaxK = 4 * kMcSteps;
constexpr int kMcRow = 68;                  // floats per channel row of the store staging (64 pixels + pad)
constexpr int kMcStageFloats = 16 * kMcRow; // per wavefront: 16 channel rows
constexpr int kMcMaxInFloats = 8192;        // largest staged input window: 32 KB

// Rows of the input window a workgroup reads: output rows oh_a .. oh_b.
__device__ __host__ __forceinline__ int mc_window_rows(int oh_a, int oh_b, int s) { return (oh_b - oh_a) * s + 3; }

__global__ __launch_bounds__(64 * kMcWaves) void k_conv_mfma(ConvArgs a, const uint32_t* __restrict__ bits,
                                                             const float* __restrict__ x,
                                                             const float* __restrict__ wt,
                                                             const float* __restrict__ bias_p, float* __restrict__ y,
                                                             int groups, int blocks_per_frame, int win) {
  extern __shared__ __align__(16) float smem[];
  float* s_w = smem;                                  // [k][64]
  float* s_b = s_w + kMcMaxK * 64;                    // [64]
  float* s_stage = s_b + 64;                          // kMcWaves x [16][kMcRow]
  float* s_in = s_stage + kMcWaves * kMcStageFloats;  // [ci][window row][w_in + 2], zero halo; win floats
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  const int grp = blockIdx.x % groups;
  const int co0 = grp * 64;
  const int blk = blockIdx.x / groups;
  const int64_t frame = blk / blocks_per_frame;
  const int pw0 = (blk - (int)(frame * blocks_per_frame)) * kMcPixels;  // first pixel of the workgroup
  const int K = a.c_in * 9;
  const int oh_a = pw0 / a.w_out;
  const int oh_b = (min(pw0 + kMcPixels, a.hw_out) - 1) / a.w_out;
  const int rows = mc_window_rows(oh_a, oh_b, a.s);
  const int ih_a = oh_a * a.s - 1;
  const int wp = a.w_in + 2;
  const int plane = rows * wp;
  const int nin = a.c_in * plane;

  // Stage the masked input window, the weights and the bias: every load of a
  // thread is issued before its first LDS write.
  {
    constexpr int kPer = kMcMaxInFloats / (64 * kMcWaves);  // up to 32 window elements per thread
    float v[kPer];
    const float* xf = x + frame * (int64_t)a.c_in * a.hw_in;
    const uint32_t* bf = bits + frame * (int64_t)a.hw_in * a.cwp;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = (int)threadIdx.x + j * 64 * kMcWaves;
      if (j * 64 * kMcWaves >= win) break;  // uniform: the window is smaller
      const int ci = i / plane, rem = i - (i / plane) * plane;
      const int r = rem / wp, c = rem - (rem / wp) * wp;
      const int ih = ih_a + r, iw = c - 1;
      const bool in = i < nin && ih >= 0 && ih < a.h_in && iw >= 0 && iw < a.w_in;
      float xv = 0.f;
      if (in) {
        const int pix = ih * a.w_in + iw;
        xv = ((bf[(int64_t)pix * a.cwp + (ci >> 5)] >> (ci & 31)) & 1u) ? xf[(int64_t)ci * a.hw_in + pix] : 0.f;
      }
      v[j] = xv;
    }
    float wv[kMcMaxK * 64 / (64 * kMcWaves)];
#pragma unroll
    for (int j = 0; j < kMcMaxK * 64 / (64 * kMcWaves); ++j) {
      const int i = (int)threadIdx.x + j * 64 * kMcWaves;
      const int k = i >> 6, c = co0 + (i & 63);
      wv[j] = (k < K && c < a.c_out) ? wt[(int64_t)k * a.c_out + c] : 0.f;
    }
    const float bv = (threadIdx.x < 64 && bias_p != nullptr && co0 + (int)threadIdx.x < a.c_out)
                         ? bias_p[co0 + threadIdx.x] : 0.f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = (int)threadIdx.x + j * 64 * kMcWaves;
      if (j * 64 * kMcWaves >= win) break;
      if (i < nin) s_in[i] = v[j];
    }
#pragma unroll
    for (int j = 0; j < kMcMaxK * 64 / (64 * kMcWaves); ++j) s_w[(int)threadIdx.x + j * 64 * kMcWaves] = wv[j];
    if (threadIdx.x < 64) s_b[threadIdx.x] = bv;
  }
  __syncthreads();

  const int p0 = pw0 + 64 * wave;  // this wavefront's first pixel
  if (p0 >= a.hw_out) return;      // no barrier below
  const int pl = lane & 15, kl = lane >> 4;
  // Window offset of this lane's pixel (tap (0, 0)) in each pixel block.
  int wofs[4];
#pragma unroll
  for (int pb = 0; pb < 4; ++pb) {
    const int p = min(p0 + 16 * pb + pl, a.hw_out - 1);
    const int oh = p / a.w_out, ow = p - (p / a.w_out) * a.w_out;
    wofs[pb] = (oh * a.s - 1 - ih_a) * wp + ow * a.s;
  }
  mc_f32x4 acc[4][4];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) {
    const float b = s_b[16 * cb + pl];
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) acc[pb][cb] = mc_f32x4{b, b, b, b};
  }
  const int nsteps = (K + 3) / 4;
#pragma unroll
  for (int st = 0; st < kMcSteps; ++st) {
    if (st < nsteps) {
      const int k = st * 4 + kl;
      const bool kin = k < K;
      const int kc = kin ? k : 0;  // the window address stays inside it
      const int ci = kc / 9, tap = kc - (kc / 9) * 9;
      const int kofs = ci * plane + (tap / 3) * wp + tap % 3;
      float av[4], bv[4];
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) av[pb] = kin ? s_in[kofs + wofs[pb]] : 0.f;
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) bv[cb] = s_w[k * 64 + 16 * cb + pl];
#pragma unroll
      for (int pb = 0; pb < 4; ++pb)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
          acc[pb][cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[pb], bv[cb], acc[pb][cb], 0, 0, 0);
    }
  }

  float* stage = s_stage + wave * kMcStageFloats;
  const int q = lane & 15, cq = lane >> 4;
  const int p = p0 + 4 * q;
  const int npx = a.hw_out - p;
  const bool vec_ok = (a.hw_out & 3) == 0;
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) {
#pragma unroll
    for (int pb = 0; pb < 4; ++pb)
      *reinterpret_cast<mc_f32x4*>(stage + pl * kMcRow + 16 * pb + 4 * kl) = acc[pb][cb];
    // Lanes read rows other lanes wrote: a wavefront-scope release / acquire
    // around the wave barrier (the region is this wavefront's own).
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // Lane l: channel 16 cb + 4 i + l / 16, pixels 4 (l % 16) .. +3.
    mc_f32x4 out[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = *reinterpret_cast<const mc_f32x4*>(stage + (4 * i + cq) * kMcRow + 4 * q);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the next block's writes after these reads
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int co = co0 + 16 * cb + 4 * i + cq;
      if (co >= a.c_out || npx <= 0) continue;
      float* yp = y + (frame * a.c_out + co) * (int64_t)a.hw_out + p;
      if (vec_ok && npx >= 4) {
        // Written once and never read back by this kernel.
        __builtin_nontemporal_store(out[i], reinterpret_cast<mc_f32x4*>(yp));
      } else {
        yp[0] = out[i].x;
        if (npx > 1) yp[1] = out[i].y;
        if (npx > 2) yp[2] = out[i].z;
        if (npx > 3) yp[3] = out[i].w;
      }
    }
  }
}

// LDS besides the input window: weights, bias, store staging.
constexpr size_t kMcFixedLds = (size_t)(kMcMaxK * 64 + 64 + kMcWaves * kMcStageFloats) * sizeof(float);

// Largest input window (floats) of a workgroup's 256 output pixels: their
// output rows, the stride-spaced input rows they read, all C_in planes, a
// zero halo.
int64_t mc_window_floats(const ConvArgs& a) {
  const int span = (kMcPixels - 1) / a.w_out + 2;  // output rows 256 consecutive pixels can touch
  return (int64_t)a.c_in * mc_window_rows(0, span - 1, a.s) * (a.w_in + 2);
}

}  // namespace

// The input window must fit the 32 KB staging area.
bool mfma_conv_applicable(const ConvArgs& a) {
  if (a.k != 3 || a.c_in * 9 > kMcMaxK || a.cwp != 1 || a.w_out < 1) return false;
  return mc_window_floats(a) <= kMcMaxInFloats;
}

int launch_conv_mfma(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  if (in_dtype != SF_F32 || out_dtype != SF_F32) return (int)hipErrorInvalidValue;
  timing_begin(K_MFMA_CONV, stream);
  const int groups = (a.c_out + 63) / 64;
  const int bpf = (a.hw_out + kMcPixels - 1) / kMcPixels;
  const int64_t blocks = a.n * (int64_t)bpf * groups;
  const int win = (int)mc_window_floats(a);
  const size_t lds = kMcFixedLds + (size_t)win * sizeof(float);
  const int e = set_lds_limit_once<k_conv_mfma>((int)(kMcFixedLds + kMcMaxInFloats * sizeof(float)));
  if (e != (int)hipSuccess) {
    timing_end(K_MFMA_CONV, stream);
    return e;
  }
  hipLaunchKernelGGL(k_conv_mfma, dim3((unsigned)blocks), dim3(64 * kMcWaves), lds, stream, a, a.bits,
                     static_cast<const float*>(a.x), a.wt, a.bias, static_cast<float*>(a.y), groups, bpf, win);
  const int rc = (int)hipGetLastError();
  timing_end(K_MFMA_CONV, stream);
  return rc;
}

}  // namespace sf
