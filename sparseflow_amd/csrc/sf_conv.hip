// Stage 2 of the spike-sparse convolution: deterministic gather conv over the
// Stage-1 bitmap, and the fused conv + multi-step LIF kernel.
//
// Work unit: one wavefront owns a group of 64 consecutive output pixels of
// one frame (row-major, so the group's outputs are contiguous per channel in
// NCHW) and produces every output channel for them.
//
//   Phase A (lane = pixel).  Each lane reads the bitmap words of its k*k
//     receptive-field pixels and counts its active (ci, kh, kw) taps; a
//     wavefront prefix sum places every pixel's entries, and each lane then
//     writes one entry per active tap -- the byte offset of weight row
//     (ci*k + kh)*k + kw and its pixel slot, packed as offset << 6 | slot --
//     into a per-wavefront LDS list.  The list is sorted by pixel, and by
//     (kh, kw, ci) within a pixel.
//   Phase B (lane = output channel).  The wavefront walks the list linearly
//     in blocks of 16 entries held in scalar registers: 16 independent
//     weight-row buffer loads are issued before any is consumed, then summed
//     in list order into a running per-pixel accumulator (restarting from the
//     bias at each pixel) that is parked in the pixel's LDS stage slot.  Binary spikes add the weight
//     itself; chunks flagged non-binary FMA value * weight, the value read
//     from x.  The stage is then written out transposed (lane = pixel), so
//     NCHW stores are contiguous runs per channel.
//
// Every output element is bias + its taps summed by one wavefront in a fixed
// order: results are deterministic and identical from run to run.  No
// atomics.  This
// replaces the reference's per-tile grouped tl.dot kernels
// (Kernels/conv2d.py:237-361, 364-460, 564-886) and the fused conv-LIF kernels
// (Kernels/fused_conv_lif.py:63-303).
#include "sf_internal.h"

namespace sf {

namespace {

constexpr int kBlock = 16;  // weight-row loads in flight per wavefront

struct WaveLds {
  int32_t* list;  // [cap] packed entries
  float* stage;   // [64 channels][ld] per-pixel results
};

__device__ __forceinline__ WaveLds wave_lds(char* smem, const ConvArgs& a, int wave) {
  char* base = smem + (size_t)wave * a.wave_lds;
  WaveLds w;
  w.list = reinterpret_cast<int32_t*>(base);
  w.stage = reinterpret_cast<float*>(base + (size_t)a.cap * 4);
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
template <int K>
__device__ __forceinline__ void decode_taps(const ConvArgs& a, const uint32_t* fb, int oh, int ow, int slot, int pos,
                                            int32_t* list) {
#pragma unroll
  for (int kh = 0; kh < K; ++kh) {
    const int ih = oh * a.s - a.p + kh;
    if (ih < 0 || ih >= a.h_in) continue;
#pragma unroll
    for (int kw = 0; kw < K; ++kw) {
      const int iw = ow * a.s - a.p + kw;
      if (iw < 0 || iw >= a.w_in) continue;
      const uint32_t* wp = fb + ((int64_t)ih * a.w_in + iw) * a.cwp;
      for (int cw = 0; cw < a.cwp; ++cw) {
        uint32_t wd = wp[cw];
        while (wd != 0u) {
          const int b = __builtin_ctz(wd);
          wd &= wd - 1u;
          const uint32_t row = (uint32_t)(((cw * 32 + b) * K + kh) * K + kw);
          if (pos < a.cap) list[pos] = (int32_t)(((row * (uint32_t)a.c_out * 4u) << 6) | (uint32_t)slot);
          ++pos;
        }
      }
    }
  }
}

// Buffer resource over the weight matrix: raw (stride 0) dword loads, so a
// weight-row load is one buffer_load with the row's byte offset in soffset
// (scalar) and the lane's column offset in voffset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t weight_rsrc(const ConvArgs& a) {
  const int bytes = a.c_in * a.k * a.k * a.c_out * 4;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.wt), (short)0, bytes, 0x00020000);
}

// Phase B: sum the weight rows of list entries [i0, i1) (sorted by slot) for
// output channels co[j] into the LDS stage: stage_row[j][slot] ends as the
// bias plus the slot's entries in list ((kh, kw, ci)) order.  The caller
// initialises the stage with the bias for slots without entries.
// Entries are read in blocks of 16 into scalar registers and all 16
// weight-row loads are issued before the first is consumed; pixel (slot)
// changes are uniform scalar branches, so the per-entry vector work is one
// add per output channel.  Out-of-range channels read a clamped in-bounds
// column whose result is never stored.  pin_base (per lane = slot) is the
// flat input index of the slot's receptive-field origin (value path only).
// One block of up to kBlock entries starting at list[ib]; FULL blocks have
// exactly kBlock entries (no tail handling).  State (acc, cur) carries over.
template <int K, int CPL, bool VALUE, bool FULL, typename TIn>
__device__ __forceinline__ void walk_block(const ConvArgs& a, const __amdgpu_buffer_rsrc_t& wr, const int32_t* list,
                                           int ib, int n, const int (&col_bytes)[CPL], const float (&bias)[CPL],
                                           float* const (&stage_row)[CPL], const TIn* xf, int pin_base,
                                           float (&acc)[CPL], int& cur) {
  int ent[kBlock];
#pragma unroll
  for (int q = 0; q < kBlock; ++q) ent[q] = __builtin_amdgcn_readfirstlane(list[ib + (FULL ? q : min(q, n - 1))]);
  float wv[kBlock][CPL];
#pragma unroll
  for (int q = 0; q < kBlock; ++q) {
    const int off = (int)((uint32_t)ent[q] >> 6);
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      wv[q][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wr, col_bytes[j], off, 0));
  }
  float xv[kBlock];
  if (VALUE) {
#pragma unroll
    for (int q = 0; q < kBlock; ++q) {
      const int row = (int)(((uint32_t)ent[q] >> 6) / ((uint32_t)a.c_out * 4u));
      const int slot = ent[q] & 63;
      const int ci = row / (K * K);
      const int tap = row - ci * (K * K);
      const int kh = tap / K;
      const int kw = tap - kh * K;
      const int pin = __builtin_amdgcn_readlane(pin_base, slot) + kh * a.w_in + kw;
      xv[q] = to_f32<TIn>(xf[(int64_t)ci * a.hw_in + pin]);
    }
  }
#pragma unroll
  for (int q = 0; q < kBlock; ++q) {
    if (FULL || q < n) {
      const int slot = ent[q] & 63;
      if (slot != cur) {
        if (cur >= 0) {
#pragma unroll
          for (int j = 0; j < CPL; ++j) stage_row[j][cur] = acc[j];
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) acc[j] = bias[j];
        cur = slot;
      }
#pragma unroll
      for (int j = 0; j < CPL; ++j) acc[j] = VALUE ? fmaf(xv[q], wv[q][j], acc[j]) : acc[j] + wv[q][j];
    }
  }
}

template <int K, int CPL, bool VALUE, typename TIn>
__device__ __forceinline__ void walk_entries(const ConvArgs& a, const int32_t* list, int i0, int i1,
                                             const int (&co_eff)[CPL], const float (&bias)[CPL],
                                             float* const (&stage_row)[CPL], const TIn* xf, int pin_base) {
  const __amdgpu_buffer_rsrc_t wr = weight_rsrc(a);
  int col_bytes[CPL];
  float acc[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    col_bytes[j] = co_eff[j] * 4;
    acc[j] = bias[j];
  }
  int cur = -1;
  int ib = i0;
  for (; ib + kBlock <= i1; ib += kBlock)
    walk_block<K, CPL, VALUE, true, TIn>(a, wr, list, ib, kBlock, col_bytes, bias, stage_row, xf, pin_base, acc, cur);
  if (ib < i1)
    walk_block<K, CPL, VALUE, false, TIn>(a, wr, list, ib, i1 - ib, col_bytes, bias, stage_row, xf, pin_base, acc,
                                          cur);
  if (cur >= 0) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) stage_row[j][cur] = acc[j];
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
  constexpr int LD = 33;  // stage row stride (32 pixel slots + 1 pad word)
  constexpr int CH = 64 * CPL;

  const int64_t frame = gidx / a.groups_per_frame;
  const int g = (int)(gidx - frame * a.groups_per_frame);
  const int pix0 = g * kWave;
  const int nvalid = min(kWave, a.hw_out - pix0);
  const int pix = pix0 + lane;
  const bool pvalid = lane < nvalid;
  const int oh = pix / a.w_out;
  const int ow = pix - oh * a.w_out;
  const int pin_base = (oh * a.s - a.p) * a.w_in + (ow * a.s - a.p);

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
    if (lane >= s && lane < e) decode_taps<K>(a, fb, oh, ow, lane, excl - base, w.list);
    wave_lds_sync();

    for (int c0 = 0; c0 < a.c_out; c0 += CH) {
      int co_eff[CPL];
      float bias[CPL];
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int co = c0 + lane + 64 * j;
        co_eff[j] = min(co, a.c_out - 1);
        bias[j] = (a.bias != nullptr && co < a.c_out) ? a.bias[co] : 0.f;
      }
      // Halves of 32 pixel slots share one stage.
      for (int h0 = s; h0 < e;) {
        const int sb = h0 & ~31;
        const int h1 = min(e, sb + 32);
        const int i0 = (h0 > 0 ? __builtin_amdgcn_readlane(incl, h0 - 1) : 0) - base;
        const int i1 = min(__builtin_amdgcn_readlane(incl, h1 - 1) - base, a.cap);
        float* stage_row[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          stage_row[j] = w.stage + (lane + 64 * j) * LD - sb;
          for (int p = h0; p < h1; ++p) stage_row[j][p] = bias[j];
        }
        if (value_path) {
          walk_entries<K, CPL, true, TIn>(a, w.list, i0, i1, co_eff, bias, stage_row, xf, pin_base);
        } else {
          walk_entries<K, CPL, false, TIn>(a, w.list, i0, i1, co_eff, bias, stage_row, xf, pin_base);
        }
        wave_lds_sync();
        // Transposed store: lanes 0-31 write channel r, lanes 32-63 channel r+1.
        const int px = sb + (lane & 31);
        if (px >= h0 && px < h1) {
          for (int r = lane >> 5; r < CH; r += 2) {
            if (c0 + r < a.c_out) yf[(int64_t)(c0 + r) * a.hw_out + px] = from_f32<TOut>(w.stage[r * LD + (px - sb)]);
          }
        }
        wave_lds_sync();
        h0 = h1;
      }
    }
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
  constexpr int LD = 65;

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
  const int pin_base = (oh * a.s - a.p) * a.w_in + (ow * a.s - a.p);

  float v[64];
#pragma unroll
  for (int c = 0; c < 64; ++c) {
    const int co = cb + c;
    v[c] = (a.v_init != nullptr && pvalid && co < a.c_out)
               ? a.v_init[(n * a.c_out + co) * (int64_t)a.hw_out + pix]
               : 0.f;
  }
  const int co = cb + lane;
  const int co_eff[1] = {min(co, a.c_out - 1)};
  const float bias[1] = {(a.bias != nullptr && co < a.c_out) ? a.bias[co] : 0.f};
  const float tau = a.tau, vth = a.v_th, vr = a.hard_reset ? a.v_reset : 0.f;
  float* const stage_row[1] = {w.stage + lane * LD};

  for (int t = 0; t < a.T; ++t) {
    const int64_t frame = (int64_t)t * a.n + n;
    const bool value_path = group_value_path<K>(a, frame, pix0, nvalid);
    const uint32_t* fb = a.bits + frame * (int64_t)a.hw_in * a.cwp;
    const TIn* xf = static_cast<const TIn*>(a.x) + frame * (int64_t)a.c_in * a.hw_in;

    const int cnt = count_taps<K>(a, fb, pvalid, oh, ow);
    const int incl = wave_inclusive_scan(cnt);
    const int excl = incl - cnt;

    for (int p = 0; p < nvalid; ++p) stage_row[0][p] = bias[0];
    int s = 0;
    while (s < nvalid) {
      const int base = s > 0 ? __builtin_amdgcn_readlane(incl, s - 1) : 0;
      const uint64_t fit = __ballot(lane >= s && lane < nvalid && (incl - base) <= a.cap);
      int e = s + __popcll(fit);
      if (e == s) e = s + 1;
      if (lane >= s && lane < e) decode_taps<K>(a, fb, oh, ow, lane, excl - base, w.list);
      wave_lds_sync();
      const int i1 = min(__builtin_amdgcn_readlane(incl, e - 1) - base, a.cap);
      if (value_path) {
        walk_entries<K, 1, true, TIn>(a, w.list, 0, i1, co_eff, bias, stage_row, xf, pin_base);
      } else {
        walk_entries<K, 1, false, TIn>(a, w.list, 0, i1, co_eff, bias, stage_row, xf, pin_base);
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
        const float cur = w.stage[c * LD + lane];
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

template <typename TIn, typename TOut>
int launch_conv_t(const ConvArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.total_groups + a.waves_per_block - 1) / a.waves_per_block;
  if (blocks == 0) return (int)hipSuccess;
  const size_t lds = (size_t)a.waves_per_block * a.wave_lds;
  const dim3 grid((unsigned)blocks), block(64 * a.waves_per_block);
  const bool wide = a.c_out >= 128;
#define SF_LAUNCH_CONV(KK, CC)                                   \
  do {                                                           \
    constexpr auto kern = k_conv_gather<TIn, TOut, KK, CC>;      \
    const int e = set_lds_limit_once<kern>(kMaxLdsBytes);        \
    if (e != (int)hipSuccess) return e;                          \
    hipLaunchKernelGGL(kern, grid, block, lds, stream, a);       \
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
    constexpr auto kern = k_conv_lif<TIn, TOut, 3>;
    const int e = set_lds_limit_once<kern>(kMaxLdsBytes);
    if (e != (int)hipSuccess) return e;
    hipLaunchKernelGGL(kern, grid, block, lds, stream, a);
  } else {
    constexpr auto kern = k_conv_lif<TIn, TOut, 1>;
    const int e = set_lds_limit_once<kern>(kMaxLdsBytes);
    if (e != (int)hipSuccess) return e;
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
  int cap = per_pixel_max > 1024 ? per_pixel_max : 1024;
  a.cap = (cap + kBlock - 1) / kBlock * kBlock;
  a.fl = lif ? 64 : 32;
  const int cpl = (!lif && a.c_out >= 128) ? 2 : 1;
  const int stage = 64 * cpl * (lif ? 65 : 33) * 4;
  a.wave_lds = ((a.cap * 4 + stage) + 15) / 16 * 16;
  // Blocks of up to 4 wavefronts; pick the size whose whole blocks keep the
  // most wavefronts resident within one CU's LDS (ties -> larger blocks).
  int per_cu = kMaxLdsBytes / a.wave_lds;
  if (per_cu < 1) per_cu = 1;
  int best = 1, best_res = per_cu;
  for (int wpb = 2; wpb <= 4 && wpb <= per_cu; ++wpb) {
    const int res = (per_cu / wpb) * wpb;
    if (res >= best_res) {
      best = wpb;
      best_res = res;
    }
  }
  a.waves_per_block = best;
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
