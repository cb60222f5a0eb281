// Stage 2 of the spike-sparse convolution: deterministic gather conv over the
// Stage-1 bitmap, and the fused conv + multi-step LIF kernel.
//
// Work unit: one wavefront owns a group of 64 consecutive output pixels of
// one frame (row-major, so the group's outputs are contiguous per channel in
// NCHW) and produces every output channel for them.
//
//   Phase A (lane = pixel).  Each lane reads the bitmap words of its k*k
//     receptive-field pixels, counts active (ci, kh, kw) taps, and after a
//     wavefront prefix sum writes one entry per active tap -- the element
//     offset of weight row (ci*k + kh)*k + kw -- into a per-wavefront LDS
//     list.  Entries of a pixel are contiguous and ascending in (kh, kw, ci).
//     Chunks flagged non-binary also store the activation value.
//   Phase B (lane = output channel).  For each pixel in turn the wavefront
//     walks that pixel's entries and adds the weight rows (binary spikes: the
//     product is the weight itself) or FMAs value * weight, starting from the
//     bias.  Results go through an LDS stage so the NCHW stores are
//     contiguous runs per channel.
//
// No atomics: every output element is summed by one wavefront in a fixed
// order, so results are deterministic.  This replaces the reference's
// per-tile grouped tl.dot kernels (Kernels/conv2d.py:237-361, 364-460,
// 564-886) and the fused conv-LIF kernels (Kernels/fused_conv_lif.py:63-303).
#include "sf_internal.h"

namespace sf {

namespace {

// Per-wavefront LDS layout: [cap] int32 entries | [cap] f32 values | stage.
struct WaveLds {
  int32_t* list;
  float* vals;
  float* stage;
};

__device__ __forceinline__ WaveLds wave_lds(char* smem, const ConvArgs& a, int wave) {
  char* base = smem + (size_t)wave * a.wave_lds;
  WaveLds w;
  w.list = reinterpret_cast<int32_t*>(base);
  w.vals = reinterpret_cast<float*>(base + (size_t)a.cap * 4);
  w.stage = reinterpret_cast<float*>(base + (size_t)a.cap * 8);
  return w;
}

// OR of the non-binary chunk flags that cover the input rows read by the
// output pixels [pix0, pix0 + nvalid) of `frame`.
template <int K>
__device__ __forceinline__ bool group_value_path(const ConvArgs& a, int64_t frame, int pix0, int nvalid) {
  const int oh_a = pix0 / a.w_out;
  const int oh_b = (pix0 + nvalid - 1) / a.w_out;
  const int ih_a = max(0, oh_a * a.s - a.p);
  const int ih_b = min(a.h_in - 1, oh_b * a.s - a.p + K - 1);
  if (ih_b < ih_a) return false;
  const int64_t c_a = ((int64_t)ih_a * a.w_in) / a.chunk;
  const int64_t c_b = ((int64_t)ih_b * a.w_in + a.w_in - 1) / a.chunk;
  const uint32_t* fl = a.flags + frame * a.chunks_per_frame;
  uint32_t f = 0u;
  for (int64_t q = c_a; q <= c_b; ++q) f |= fl[q];
  return f != 0u;
}

// Phase A, pass 1: active taps of this lane's output pixel.
template <int K>
__device__ __forceinline__ int count_taps(const ConvArgs& a, const uint32_t* fb, bool pvalid, int oh, int ow) {
  int cnt = 0;
  if (!pvalid) return 0;
#pragma unroll
  for (int kh = 0; kh < K; ++kh) {
    const int ih = oh * a.s - a.p + kh;
    if (ih < 0 || ih >= a.h_in) continue;
#pragma unroll
    for (int kw = 0; kw < K; ++kw) {
      const int iw = ow * a.s - a.p + kw;
      if (iw < 0 || iw >= a.w_in) continue;
      const uint32_t* wp = fb + ((int64_t)ih * a.w_in + iw) * a.cwp;
      for (int cw = 0; cw < a.cwp; ++cw) cnt += __popc(wp[cw]);
    }
  }
  return cnt;
}

// Phase A, pass 2: write this lane's entries starting at list[pos].
template <int K, typename TIn>
__device__ __forceinline__ void decode_taps(const ConvArgs& a, const uint32_t* fb, const TIn* xf, int oh, int ow,
                                            int pos, bool value_path, const WaveLds& w) {
#pragma unroll
  for (int kh = 0; kh < K; ++kh) {
    const int ih = oh * a.s - a.p + kh;
    if (ih < 0 || ih >= a.h_in) continue;
#pragma unroll
    for (int kw = 0; kw < K; ++kw) {
      const int iw = ow * a.s - a.p + kw;
      if (iw < 0 || iw >= a.w_in) continue;
      const int64_t pin = (int64_t)ih * a.w_in + iw;
      const uint32_t* wp = fb + pin * a.cwp;
      for (int cw = 0; cw < a.cwp; ++cw) {
        uint32_t wd = wp[cw];
        while (wd != 0u) {
          const int b = __builtin_ctz(wd);
          wd &= wd - 1u;
          const int ci = cw * 32 + b;
          if (pos < a.cap) {
            w.list[pos] = ((ci * K + kh) * K + kw) * a.c_out;
            if (value_path) w.vals[pos] = to_f32<TIn>(xf[(int64_t)ci * a.hw_in + pin]);
          }
          ++pos;
        }
      }
    }
  }
}

// Phase B inner loop: acc[j] (+)= sum over entries [st, st+ct) of the weight
// rows at output channel co_j, in entry order.
template <int CPL, bool VALUE>
__device__ __forceinline__ void accumulate(const ConvArgs& a, const WaveLds& w, int st, int ct, int c0, int lane,
                                           float (&acc)[CPL]) {
  const int32_t* lp = w.list + st;
  const float* vp = w.vals + st;
  const float* wt = a.wt;
  bool co_ok[CPL];
  int co[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    co[j] = c0 + lane + 64 * j;
    co_ok[j] = co[j] < a.c_out;
  }
  int k = 0;
  for (; k + 8 <= ct; k += 8) {
    int r[8];
    float v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) r[q] = lp[k + q];
    if (VALUE) {
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = vp[k + q];
    }
    float wv[8][CPL];
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int j = 0; j < CPL; ++j) wv[q][j] = co_ok[j] ? wt[r[q] + co[j]] : 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int j = 0; j < CPL; ++j) acc[j] = VALUE ? fmaf(v[q], wv[q][j], acc[j]) : acc[j] + wv[q][j];
  }
  for (; k < ct; ++k) {
    const int r = lp[k];
    const float v = VALUE ? vp[k] : 1.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const float wv = co_ok[j] ? wt[r + co[j]] : 0.f;
      acc[j] = VALUE ? fmaf(v, wv, acc[j]) : acc[j] + wv;
    }
  }
}

template <typename TIn, typename TOut, int K, int CPL>
__global__ __launch_bounds__(256) void k_conv_gather(ConvArgs a) {
  extern __shared__ __align__(16) char smem[];
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const int64_t gidx = (int64_t)blockIdx.x * a.waves_per_block + wave;
  if (gidx >= a.total_groups) return;  // wavefronts never wait on each other
  const WaveLds w = wave_lds(smem, a, wave);
  const int flp = a.fl + 1;

  const int64_t frame = gidx / a.groups_per_frame;
  const int g = (int)(gidx - frame * a.groups_per_frame);
  const int pix0 = g * kWave;
  const int nvalid = min(kWave, a.hw_out - pix0);
  const int pix = pix0 + lane;
  const bool pvalid = lane < nvalid;
  const int oh = pix / a.w_out;
  const int ow = pix - oh * a.w_out;

  const bool value_path = group_value_path<K>(a, frame, pix0, nvalid);
  const uint32_t* fb = a.bits + frame * (int64_t)a.hw_in * a.cwp;
  const TIn* xf = static_cast<const TIn*>(a.x) + frame * (int64_t)a.c_in * a.hw_in;
  TOut* yf = static_cast<TOut*>(a.y) + frame * (int64_t)a.c_out * a.hw_out + pix0;

  const int cnt = count_taps<K>(a, fb, pvalid, oh, ow);
  const int incl = wave_inclusive_scan(cnt);
  const int excl = incl - cnt;

  int s = 0;
  while (s < nvalid) {
    // Batch [s, e): the longest run of pixels whose entries fit the list.
    const int base = s > 0 ? __builtin_amdgcn_readlane(incl, s - 1) : 0;
    const uint64_t fit = __ballot(lane >= s && lane < nvalid && (incl - base) <= a.cap);
    int e = s + __popcll(fit);
    if (e == s) e = s + 1;
    if (lane >= s && lane < e) decode_taps<K, TIn>(a, fb, xf, oh, ow, excl - base, value_path, w);
    wave_lds_sync();

    for (int c0 = 0; c0 < a.c_out; c0 += 64 * CPL) {
      float bias[CPL];
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int co = c0 + lane + 64 * j;
        bias[j] = (a.bias != nullptr && co < a.c_out) ? a.bias[co] : 0.f;
      }
      int fs = s;
      for (int p = s; p < e; ++p) {
        const int st = __builtin_amdgcn_readlane(excl, p) - base;
        const int ct = min(__builtin_amdgcn_readlane(cnt, p), a.cap - st);
        float acc[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) acc[j] = bias[j];
        if (value_path) {
          accumulate<CPL, true>(a, w, st, ct, c0, lane, acc);
        } else {
          accumulate<CPL, false>(a, w, st, ct, c0, lane, acc);
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) w.stage[(lane + 64 * j) * flp + (p - fs)] = acc[j];
        if (p - fs == a.fl - 1 || p == e - 1) {
          wave_lds_sync();
          const int m = p - fs + 1;
          const int rows_per = kWave / a.fl;
          const int ro = lane / a.fl;
          const int px = lane - ro * a.fl;
          if (px < m) {
            for (int r = ro; r < 64 * CPL; r += rows_per) {
              const int co = c0 + r;
              if (co < a.c_out) yf[(int64_t)co * a.hw_out + fs + px] = from_f32<TOut>(w.stage[r * flp + px]);
            }
          }
          wave_lds_sync();
          fs = p + 1;
        }
      }
    }
    wave_lds_sync();
    s = e;
  }
}

// Fused conv + LIF.  One wavefront owns 64 pixels x 64 output channels of one
// sample n and runs all T steps; the membrane lives in 64 VGPRs per lane
// (lane = pixel) between steps.
template <typename TIn, typename TOut, int K>
__global__ __launch_bounds__(256) void k_conv_lif(ConvArgs a) {
  extern __shared__ __align__(16) char smem[];
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const int nco = (a.c_out + 63) / 64;
  const int64_t widx = (int64_t)blockIdx.x * a.waves_per_block + wave;
  if (widx >= a.total_groups * nco) return;
  const WaveLds w = wave_lds(smem, a, wave);
  constexpr int FLP = 65;

  const int64_t gidx = widx / nco;
  const int cb = (int)(widx - gidx * nco) * 64;
  const int64_t n = gidx / a.groups_per_frame;
  const int g = (int)(gidx - n * a.groups_per_frame);
  const int pix0 = g * kWave;
  const int nvalid = min(kWave, a.hw_out - pix0);
  const int pix = pix0 + lane;
  const bool pvalid = lane < nvalid;
  const int oh = pix / a.w_out;
  const int ow = pix - oh * a.w_out;

  float v[64];
#pragma unroll
  for (int c = 0; c < 64; ++c) {
    const int co = cb + c;
    v[c] = (a.v_init != nullptr && pvalid && co < a.c_out)
               ? a.v_init[(n * a.c_out + co) * (int64_t)a.hw_out + pix]
               : 0.f;
  }
  const float bias = (a.bias != nullptr && cb + lane < a.c_out) ? a.bias[cb + lane] : 0.f;
  const float tau = a.tau, vth = a.v_th, vr = a.hard_reset ? a.v_reset : 0.f;

  for (int t = 0; t < a.T; ++t) {
    const int64_t frame = (int64_t)t * a.n + n;
    const bool value_path = group_value_path<K>(a, frame, pix0, nvalid);
    const uint32_t* fb = a.bits + frame * (int64_t)a.hw_in * a.cwp;
    const TIn* xf = static_cast<const TIn*>(a.x) + frame * (int64_t)a.c_in * a.hw_in;

    const int cnt = count_taps<K>(a, fb, pvalid, oh, ow);
    const int incl = wave_inclusive_scan(cnt);
    const int excl = incl - cnt;

    int s = 0;
    while (s < nvalid) {
      const int base = s > 0 ? __builtin_amdgcn_readlane(incl, s - 1) : 0;
      const uint64_t fit = __ballot(lane >= s && lane < nvalid && (incl - base) <= a.cap);
      int e = s + __popcll(fit);
      if (e == s) e = s + 1;
      if (lane >= s && lane < e) decode_taps<K, TIn>(a, fb, xf, oh, ow, excl - base, value_path, w);
      wave_lds_sync();
      for (int p = s; p < e; ++p) {
        const int st = __builtin_amdgcn_readlane(excl, p) - base;
        const int ct = min(__builtin_amdgcn_readlane(cnt, p), a.cap - st);
        float acc[1] = {bias};
        if (value_path) {
          accumulate<1, true>(a, w, st, ct, cb, lane, acc);
        } else {
          accumulate<1, false>(a, w, st, ct, cb, lane, acc);
        }
        w.stage[lane * FLP + p] = acc[0];
      }
      wave_lds_sync();
      s = e;
    }

    // LIF epilogue, lane = pixel; same operation order as the module's torch
    // path (Ops/sparse_fused_conv_lif.py:283-292).
    TOut* sp_out = static_cast<TOut*>(a.y) + (frame * a.c_out + cb) * (int64_t)a.hw_out + pix;
#pragma unroll
    for (int c = 0; c < 64; ++c) {
      if (cb + c < a.c_out) {
        const float cur = w.stage[c * FLP + lane];
        const float vp = v[c];
        const float h = a.decay_input ? vp + (cur - (vp - vr)) / tau : (vp - (vp - vr) / tau) + cur;
        const bool spike = h >= vth;
        const float vn = a.hard_reset ? (spike ? a.v_reset : h) : h - (spike ? vth : 0.f);
        v[c] = vn;
        if (pvalid) sp_out[(int64_t)c * a.hw_out] = from_f32<TOut>(spike ? 1.f : 0.f);
      }
    }
    wave_lds_sync();
  }

  if (pvalid) {
    float* vo = a.v_out + (n * a.c_out + cb) * (int64_t)a.hw_out + pix;
#pragma unroll
    for (int c = 0; c < 64; ++c)
      if (cb + c < a.c_out) vo[(int64_t)c * a.hw_out] = v[c];
  }
}

// Raise the dynamic-LDS ceiling of a kernel to the full 160 KB of a gfx950
// CU (the default limit is 64 KB).  Called once per instantiation.
template <typename K_t>
void allow_full_lds(K_t kernel) {
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            kMaxLdsBytes);
}

template <typename TIn, typename TOut>
int launch_conv_t(const ConvArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.total_groups + a.waves_per_block - 1) / a.waves_per_block;
  if (blocks == 0) return (int)hipSuccess;
  const size_t lds = (size_t)a.waves_per_block * a.wave_lds;
  const dim3 grid((unsigned)blocks), block(64 * a.waves_per_block);
  const bool wide = a.c_out >= 128;
#define SF_LAUNCH_CONV(KK, CC)                                        \
  do {                                                                \
    auto kern = k_conv_gather<TIn, TOut, KK, CC>;                     \
    static bool attr_done = false;                                    \
    if (!attr_done) { allow_full_lds(kern); attr_done = true; }       \
    hipLaunchKernelGGL(kern, grid, block, lds, stream, a);            \
  } while (0)
  if (a.k == 3) {
    if (wide) SF_LAUNCH_CONV(3, 2); else SF_LAUNCH_CONV(3, 1);
  } else {
    if (wide) SF_LAUNCH_CONV(1, 2); else SF_LAUNCH_CONV(1, 1);
  }
#undef SF_LAUNCH_CONV
  return (int)hipGetLastError();
}

template <typename TIn, typename TOut>
int launch_lif_t(const ConvArgs& a, hipStream_t stream) {
  const int nco = (a.c_out + 63) / 64;
  const int64_t waves = a.total_groups * nco;
  const int64_t blocks = (waves + a.waves_per_block - 1) / a.waves_per_block;
  if (blocks == 0) return (int)hipSuccess;
  const size_t lds = (size_t)a.waves_per_block * a.wave_lds;
  const dim3 grid((unsigned)blocks), block(64 * a.waves_per_block);
  if (a.k == 3) {
    auto kern = k_conv_lif<TIn, TOut, 3>;
    static bool attr_done = false;
    if (!attr_done) { allow_full_lds(kern); attr_done = true; }
    hipLaunchKernelGGL(kern, grid, block, lds, stream, a);
  } else {
    auto kern = k_conv_lif<TIn, TOut, 1>;
    static bool attr_done = false;
    if (!attr_done) { allow_full_lds(kern); attr_done = true; }
    hipLaunchKernelGGL(kern, grid, block, lds, stream, a);
  }
  return (int)hipGetLastError();
}

}  // namespace

void conv_geometry(ConvArgs& a, bool lif) {
  a.hw_in = a.h_in * a.w_in;
  a.hw_out = a.h_out * a.w_out;
  a.groups_per_frame = (a.hw_out + kWave - 1) / kWave;
  // The list must hold the largest possible per-pixel entry count.
  const int per_pixel_max = a.k * a.k * a.cwp * 32;
  a.cap = per_pixel_max > 512 ? per_pixel_max : 512;
  const int cpl = (!lif && a.c_out >= 128) ? 2 : 1;
  a.fl = lif ? 64 : 32;
  const int stage = 64 * cpl * (a.fl + 1) * 4;
  a.wave_lds = ((a.cap * 8 + stage) + 15) / 16 * 16;
  int wpb = kMaxLdsBytes / a.wave_lds;
  if (wpb > 4) wpb = 4;
  if (wpb < 1) wpb = 1;
  a.waves_per_block = wpb;
}

int launch_conv(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  timing_begin(K_CONV, stream);
  int rc;
  if (in_dtype == SF_F32) rc = launch_conv_t<float, float>(a, stream);
  else if (in_dtype == SF_F16) rc = out_dtype == SF_F32 ? launch_conv_t<__half, float>(a, stream)
                                                        : launch_conv_t<__half, __half>(a, stream);
  else rc = out_dtype == SF_F32 ? launch_conv_t<__hip_bfloat16, float>(a, stream)
                                : launch_conv_t<__hip_bfloat16, __hip_bfloat16>(a, stream);
  timing_end(K_CONV, stream);
  return rc;
}

int launch_conv_lif(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  timing_begin(K_LIF, stream);
  int rc;
  if (in_dtype == SF_F32) rc = launch_lif_t<float, float>(a, stream);
  else if (in_dtype == SF_F16) rc = out_dtype == SF_F32 ? launch_lif_t<__half, float>(a, stream)
                                                        : launch_lif_t<__half, __half>(a, stream);
  else rc = out_dtype == SF_F32 ? launch_lif_t<__hip_bfloat16, float>(a, stream)
                                : launch_lif_t<__hip_bfloat16, __hip_bfloat16>(a, stream);
  timing_end(K_LIF, stream);
  return rc;
}

}  // namespace sf
