// Stage 1 of the spike-sparse convolution: prescan.
//
// k_pack   streams the NCHW activation tensor once with 128-bit loads and
//          writes a channel-packed bitmap (one bit per element, 32 channels
//          per word, words of a pixel contiguous) plus one non-binary flag
//          word per pixel chunk.  Bit = f16(|x|) > f16(threshold), evaluated
//          as |x| >= cutoff (see sf_activity_cutoff).  This is the element
//          level form of the reference's fp16 cast + |.| + amax + "> thr"
//          (Kernels/conv2d.py:986; Kernels/_prescan_common.py:32-45,188).
//
// k_tiles  reads the bitmap and, per output tile, ORs the words over the
//          tile's receptive field -- the reference's RF max-pool followed by
//          the ceil-mode tile max-pool (Kernels/_prescan_common.py:167-188)
//          at group size 1 -- then derives the active-channel list (LDS
//          compaction), the group bitmask and the tile class
//          (Kernels/_prescan_common.py:48-109).
#include "sf_internal.h"

namespace sf {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// x is streamed exactly once, so its loads are marked non-temporal.
template <typename T, int VEC, bool ALIGNED>
__device__ __forceinline__ void load_vec(const T* p, float (&v)[VEC]) {
  if constexpr (ALIGNED && VEC == 4 && sizeof(T) == 4) {
    const f32x4 q = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else if constexpr (ALIGNED && VEC == 2 && sizeof(T) == 4) {
    const f32x2 q = __builtin_nontemporal_load(reinterpret_cast<const f32x2*>(p));
    v[0] = q.x; v[1] = q.y;
  } else if constexpr (ALIGNED && VEC == 4 && sizeof(T) == 2) {
    const uint2 q = *reinterpret_cast<const uint2*>(p);
    const uint32_t h[4] = {q.x & 0xffffu, q.x >> 16, q.y & 0xffffu, q.y >> 16};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      T t;
      const uint16_t b = (uint16_t)h[i];
      __builtin_memcpy(&t, &b, 2);
      v[i] = to_f32<T>(t);
    }
  } else if constexpr (ALIGNED && VEC == 2 && sizeof(T) == 2) {
    const uint32_t q = *reinterpret_cast<const uint32_t*>(p);
    const uint16_t b0 = (uint16_t)(q & 0xffffu), b1 = (uint16_t)(q >> 16);
    T t0, t1;
    __builtin_memcpy(&t0, &b0, 2);
    __builtin_memcpy(&t1, &b1, 2);
    v[0] = to_f32<T>(t0);
    v[1] = to_f32<T>(t1);
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) v[i] = to_f32<T>(p[i]);
  }
}

// One wavefront packs one chunk of 64*VEC consecutive pixels of one frame
// over a contiguous range of bitmap words (all words when csplit == 1).  A
// block has max(4, csplit) wavefronts and covers max(4, csplit)/csplit
// chunks.
// Bitmap words of a block's chunks staged in LDS when they fit, so that each
// chunk's words leave as one contiguous run of 128-bit stores instead of
// per-pixel scattered words.
constexpr int kPackStageWords = 4 * 256 * 2;  // 4 chunks x 256 pixels x 2 words (or fewer chunks x more words)

template <typename T, int VEC, bool ALIGNED>
__global__ __launch_bounds__(512) void k_pack(PackArgs a) {
  __shared__ uint32_t s_nb[8];
  __shared__ __align__(16) uint32_t s_words[kPackStageWords];
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const int csplit = a.csplit;
  const int cpb = (int)(blockDim.x >> 6) / csplit;  // chunks per block
  const int lc = wave / csplit;
  const int sp = wave - lc * csplit;
  const int64_t gchunk = (int64_t)blockIdx.x * cpb + lc;
  const bool chunk_ok = gchunk < a.total_chunks;
  const float cut = a.cutoff;
  uint32_t nb = 0;

  // Staging: chunk lc of the block owns s_words[lc * chunk * cwp ...].  (Word
  // planes need none: a lane's VEC words of one plane are consecutive.)
  const bool stage = !a.planar && cpb * 64 * VEC * a.cwp <= kPackStageWords;
  uint32_t* sw = s_words + lc * (64 * VEC) * a.cwp;
  int64_t frame = 0, chk = 0;
  if (chunk_ok) {
    frame = gchunk / a.chunks_per_frame;
    chk = gchunk - frame * a.chunks_per_frame;
    const int p0 = (int)(chk * (64 * VEC)) + lane * VEC;
    if (p0 < a.hw) {
      const int wps = a.cwp / csplit;
      const int w0 = sp * wps;
      const T* xf = static_cast<const T*>(a.x) + frame * (int64_t)a.c * a.hw + p0;
      uint32_t* bf = a.bits + (frame * a.hw + p0) * (int64_t)a.cwp;
      for (int cw = w0; cw < w0 + wps; ++cw) {
        uint32_t word[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) word[i] = 0u;
        const int cbase = cw * 32;
        if (cbase + 32 <= a.c) {
          // Full word: 32 independent loads in flight per lane.
          float v[32][VEC];
#pragma unroll
          for (int j = 0; j < 32; ++j) load_vec<T, VEC, ALIGNED>(xf + (int64_t)(cbase + j) * a.hw, v[j]);
#pragma unroll
          for (int j = 0; j < 32; ++j) {
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
              word[i] |= (fabsf(v[j][i]) >= cut ? 1u : 0u) << j;
              nb |= (v[j][i] != 0.f && v[j][i] != 1.f) ? 1u : 0u;
            }
          }
        } else if (cbase < a.c) {
          const int cnt = a.c - cbase;
          for (int j = 0; j < cnt; ++j) {
            float v[VEC];
            load_vec<T, VEC, ALIGNED>(xf + (int64_t)(cbase + j) * a.hw, v);
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
              word[i] |= (fabsf(v[i]) >= cut ? 1u : 0u) << j;
              nb |= (v[i] != 0.f && v[i] != 1.f) ? 1u : 0u;
            }
          }
        }
        if (a.planar) {
          // Plane cw of the frame: pixels p0 .. p0+VEC-1 (hw is a multiple
          // of VEC, so the VEC words are aligned to VEC words).
          uint32_t* pw = a.bits + (frame * a.cwp + cw) * (int64_t)a.hw + p0;
          if constexpr (VEC == 4) {
            *reinterpret_cast<uint4*>(pw) = make_uint4(word[0], word[1], word[2], word[3]);
          } else if constexpr (VEC == 2) {
            *reinterpret_cast<uint2*>(pw) = make_uint2(word[0], word[1]);
          } else {
            pw[0] = word[0];
          }
        } else if (stage) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) sw[(lane * VEC + i) * a.cwp + cw] = word[i];
        } else if (a.cwp == 1) {
          if constexpr (VEC == 4) {
            *reinterpret_cast<uint4*>(bf) = make_uint4(word[0], word[1], word[2], word[3]);
          } else if constexpr (VEC == 2) {
            *reinterpret_cast<uint2*>(bf) = make_uint2(word[0], word[1]);
          } else {
            bf[0] = word[0];
          }
        } else {
#pragma unroll
          for (int i = 0; i < VEC; ++i) bf[(int64_t)i * a.cwp + cw] = word[i];
        }
      }
    }
  }

  const uint64_t bal = __ballot(nb != 0u);
  if (lane == 0) s_nb[wave] = bal != 0ull ? 1u : 0u;
  __syncthreads();
  if (stage && chunk_ok) {
    // The chunk's pixels p0 .. p0+npx-1 take npx * cwp consecutive words of
    // the bitmap; its csplit wavefronts copy them out, 4 words per lane.
    const int p0 = (int)(chk * (64 * VEC));
    const int nwords = min(64 * VEC, a.hw - p0) * a.cwp;
    uint32_t* dst = a.bits + (frame * a.hw + p0) * (int64_t)a.cwp;
    const bool vec_ok = ((reinterpret_cast<uintptr_t>(dst) | (uintptr_t)nwords * 4) & 15) == 0;
    if (vec_ok) {
      for (int i = (sp * 64 + lane) * 4; i < nwords; i += csplit * 64 * 4)
        *reinterpret_cast<uint4*>(dst + i) = *reinterpret_cast<const uint4*>(sw + i);
    } else {
      for (int i = sp * 64 + lane; i < nwords; i += csplit * 64) dst[i] = sw[i];
    }
  }
  if (chunk_ok && sp == 0 && lane == 0) {
    uint32_t f = 0u;
    for (int q = 0; q < csplit; ++q) f |= s_nb[lc * csplit + q];
    a.flags[gchunk] = f;
  }
}

// Row-major prescan for the sparse linear: x [m, k] (k contiguous) -> bitmap
// [m][cwp] (bit j of word w = |x[r, 32w + j]| >= cutoff; words past the
// row's last element are zero) and one non-binary flag word per chunk of
// kLinearRowChunk rows.  One wavefront per chunk: each load covers 64
// consecutive elements of a row and one ballot turns them into two bitmap
// words.  The (row, 64-element segment) items of the chunk are taken eight
// at a time so that eight loads are in flight per lane.
// (a.n = rows, a.c = k, a.total_chunks = row chunks.)
template <typename T>
__global__ __launch_bounds__(256) void k_pack_rows(PackArgs a) {
  const int lane = lane_id();
  const int64_t chunk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (chunk >= a.total_chunks) return;  // the kernel has no block-level barrier
  const int64_t r0 = chunk * kLinearRowChunk;
  const int rows = (int)min((int64_t)kLinearRowChunk, a.n - r0);
  const int k = a.c, cwp = a.cwp;
  const int nseg = (k + 63) / 64;
  const int items = rows * nseg;
  const T* __restrict__ x = static_cast<const T*>(a.x) + r0 * (int64_t)k;
  uint32_t* __restrict__ bits = a.bits + r0 * (int64_t)cwp;
  const float cut = a.cutoff;
  uint32_t nb = 0u;
  int r = 0, sg = 0;  // item i0 = r * nseg + sg
  for (int i0 = 0; i0 < items; i0 += 8) {
    float v[8];
    int rr[8], ss[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      rr[u] = r;
      ss[u] = sg;
      const int kk = sg * 64 + lane;
      v[u] = (i0 + u < items && kk < k) ? to_f32<T>(x[(int64_t)r * k + kk]) : 0.f;
      if (++sg == nseg) { sg = 0; ++r; }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint64_t m = __ballot(fabsf(v[u]) >= cut);
      nb |= (v[u] != 0.f && v[u] != 1.f) ? 1u : 0u;
      const int w = 2 * ss[u] + lane;
      if (i0 + u < items && lane < 2 && w < cwp)
        bits[(int64_t)rr[u] * cwp + w] = lane ? (uint32_t)(m >> 32) : (uint32_t)m;
    }
  }
  if (2 * nseg < cwp) {  // padding words of the chunk's rows
    for (int i = lane; i < rows * (cwp - 2 * nseg); i += kWave) {
      const int rw = i / (cwp - 2 * nseg);
      bits[(int64_t)rw * cwp + 2 * nseg + (i - rw * (cwp - 2 * nseg))] = 0u;
    }
  }
  const uint64_t bal = __ballot(nb != 0u);
  if (lane == 0) a.flags[chunk] = bal != 0ull ? 1u : 0u;
}

// k_pack_rows with 16-byte loads (f32 rows, k % 4 == 0, x 16-byte
// aligned): each load covers 256 consecutive elements of a row, lane l
// elements 4 l .. 4 l + 3; a lane's 4-bit nibble, shifted to its place and
// OR-ed across eight lanes (three xor shuffles), is one bitmap word, stored
// by the group's first lane.  Words past the row's last element come out
// zero (the elements past k load as 0), up to 8 x ceil(k / 256) >= cwp.
__global__ __launch_bounds__(256) void k_pack_rows4(PackArgs a) {
  const int lane = lane_id();
  const int64_t chunk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (chunk >= a.total_chunks) return;  // the kernel has no block-level barrier
  const int64_t r0 = chunk * kLinearRowChunk;
  const int rows = (int)min((int64_t)kLinearRowChunk, a.n - r0);
  const int k = a.c, cwp = a.cwp;
  const int nseg = (k + 255) / 256;
  const int items = rows * nseg;
  const float* __restrict__ x = static_cast<const float*>(a.x) + r0 * (int64_t)k;
  uint32_t* __restrict__ bits = a.bits + r0 * (int64_t)cwp;
  const float cut = a.cutoff;
  uint32_t nb = 0u;
  int r = 0, sg = 0;  // item i0 = r * nseg + sg
  for (int i0 = 0; i0 < items; i0 += 8) {
    float4 v[8];
    int rr[8], ss[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      rr[u] = r;
      ss[u] = sg;
      const int kk = sg * 256 + 4 * lane;
      v[u] = (i0 + u < items && kk < k) ? *reinterpret_cast<const float4*>(x + (int64_t)r * k + kk)
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
      if (++sg == nseg) { sg = 0; ++r; }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
      uint32_t nib = 0u;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        nib |= (fabsf(e[j]) >= cut ? 1u : 0u) << j;
        nb |= (e[j] != 0.f && e[j] != 1.f) ? 1u : 0u;
      }
      uint32_t wv = nib << (4 * (lane & 7));
      wv |= __shfl_xor(wv, 1, kWave);
      wv |= __shfl_xor(wv, 2, kWave);
      wv |= __shfl_xor(wv, 4, kWave);
      const int w = 8 * ss[u] + (lane >> 3);
      if (i0 + u < items && (lane & 7) == 0 && w < cwp) bits[(int64_t)rr[u] * cwp + w] = wv;
    }
  }
  const uint64_t bal = __ballot(nb != 0u);
  if (lane == 0) a.flags[chunk] = bal != 0ull ? 1u : 0u;
}

// One wavefront per output tile.  Requires cwp <= 64 (a power of two), so
// lane l always reads word (l % cwp) of the pixels it visits.
__global__ __launch_bounds__(256) void k_tiles(TilesArgs a) {
  extern __shared__ int32_t s_list_all[];
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave;
  if (tile >= a.ntiles) return;  // the kernel has no block-level barrier
  int32_t* s_list = s_list_all + wave * a.c;

  const int gwi = (int)(tile % a.gw);
  const int64_t t2 = tile / a.gw;
  const int ghi = (int)(t2 % a.gh);
  const int64_t nn = t2 / a.gh;

  const int oh0 = ghi * a.th;
  const int oh1 = min(oh0 + a.th, a.h_out) - 1;
  const int ow0 = gwi * a.tw;
  const int ow1 = min(ow0 + a.tw, a.w_out) - 1;
  const int ih0 = max(0, oh0 * a.s - a.p);
  const int ih1 = min(a.h_in - 1, oh1 * a.s - a.p + a.k - 1);
  const int iw0 = max(0, ow0 * a.s - a.p);
  const int iw1 = min(a.w_in - 1, ow1 * a.s - a.p + a.k - 1);
  const int rh = ih1 - ih0 + 1;
  const int rw = iw1 - iw0 + 1;

  const int cwp = a.cwp;
  const int my_cw = lane & (cwp - 1);
  const int px_step = kWave / cwp;
  uint32_t acc = 0u;
  if (rh > 0 && rw > 0) {
    const int npx = rh * rw;
    const uint32_t* base = a.bits + ((nn * a.h_in + ih0) * (int64_t)a.w_in + iw0) * cwp + my_cw;
    for (int px = lane / cwp; px < npx; px += px_step) {
      const int r = px / rw;
      const int cc = px - r * rw;
      acc |= base[((int64_t)r * a.w_in + cc) * cwp];
    }
  }
  for (int off = kWave / 2; off >= cwp; off >>= 1) acc |= __shfl_xor(acc, off, kWave);
  const bool own = lane < cwp;  // lane l now holds word l of the tile mask

  if (a.ch_mask != nullptr && own) a.ch_mask[tile * cwp + lane] = acc;

  const int pc = own ? __popc(acc) : 0;
  const int incl = wave_inclusive_scan(pc);
  const int total = __shfl(incl, kWave - 1, kWave);
  if (a.ch_count != nullptr && lane == 0) a.ch_count[tile] = total;

  if (a.ch_list != nullptr) {
    // Compact: each word's owner writes its channel ids at its exclusive
    // prefix into LDS, then the wavefront copies the list out coalesced.
    int pos = incl - pc;
    uint32_t wd = own ? acc : 0u;
    while (wd != 0u) {
      const int b = __builtin_ctz(wd);
      wd &= wd - 1u;
      s_list[pos++] = lane * 32 + b;
    }
    wave_lds_sync();
    int32_t* out = a.ch_list + tile * (int64_t)a.c;
    for (int i = lane; i < total; i += kWave) out[i] = s_list[i];
  }

  if (a.ag_mask != nullptr || a.tile_class != nullptr) {
    uint32_t part = 0u;
    if (own) {
      if (a.group_size == 16) {
        part = ((acc & 0xffffu) ? 1u : 0u) << (2 * lane);
        part |= ((acc >> 16) ? 1u : 0u) << (2 * lane + 1);
      } else {
        const int wpg = a.group_size / 32;
        part = (acc != 0u ? 1u : 0u) << (lane / wpg);
      }
    }
    for (int off = kWave / 2; off >= 1; off >>= 1) part |= __shfl_xor(part, off, kWave);
    if (lane == 0) {
      const uint32_t full = a.ngroups >= 32 ? 0xffffffffu : ((1u << a.ngroups) - 1u);
      if (a.ag_mask != nullptr) a.ag_mask[tile] = (int32_t)part;
      if (a.tile_class != nullptr) a.tile_class[tile] = part == 0u ? 0 : (part == full ? 2 : 1);
    }
  }
}

template <typename T, int VEC>
int launch_pack_t(const PackArgs& a, hipStream_t stream) {
  const int wpb = a.csplit > 4 ? a.csplit : 4;
  const int cpb = wpb / a.csplit;
  const int64_t blocks = (a.total_chunks + cpb - 1) / cpb;
  if (blocks == 0) return (int)hipSuccess;
  const uintptr_t align = (uintptr_t)a.x;
  const bool aligned = (align % (sizeof(T) * VEC)) == 0;
  if (aligned) {
    hipLaunchKernelGGL((k_pack<T, VEC, true>), dim3((unsigned)blocks), dim3(64 * wpb), 0, stream, a);
  } else {
    hipLaunchKernelGGL((k_pack<T, VEC, false>), dim3((unsigned)blocks), dim3(64 * wpb), 0, stream, a);
  }
  return (int)hipGetLastError();
}

template <typename T>
int launch_pack_v(const PackArgs& a, hipStream_t stream) {
  switch (a.vec) {
    case 4: return launch_pack_t<T, 4>(a, stream);
    case 2: return launch_pack_t<T, 2>(a, stream);
    default: return launch_pack_t<T, 1>(a, stream);
  }
}

}  // namespace

int words_per_pixel(int c) {
  int w = (c + 31) / 32;
  int p = 1;
  while (p < w) p <<= 1;
  return p;
}

PackPlan make_pack_plan(int64_t n, int c, int h, int w) {
  PackPlan pl{};
  const int hw = h * w;
  pl.cwp = words_per_pixel(c);
  // Widest vector that divides the plane (so every lane's pixels are valid).
  // Channel words are split across waves first (a wave then streams one or
  // two words of 32 channels); the vector is narrowed only if the launch
  // would still leave the chip short of waves.
  const int64_t want_waves = 16384;
  int vec = (hw % 4 == 0) ? 4 : ((hw % 2 == 0) ? 2 : 1);
  auto waves_for = [&](int v, int cs) {
    const int64_t cpf = (hw + 64 * v - 1) / (64 * v);
    return n * cpf * cs;
  };
  int csplit = 1;
  while (csplit < 8 && csplit < pl.cwp && (pl.cwp / csplit > 1 || waves_for(vec, csplit) < want_waves)) csplit <<= 1;
  while (vec > 1 && waves_for(vec, csplit) < want_waves / 4) vec >>= 1;
  pl.vec = vec;
  pl.chunk = 64 * vec;
  pl.csplit = csplit;
  pl.chunks_per_frame = (hw + pl.chunk - 1) / pl.chunk;
  pl.total_chunks = n * pl.chunks_per_frame;
  return pl;
}

int launch_pack(const PackArgs& a, int dtype, hipStream_t stream) {
  timing_begin(K_PACK, stream);
  int rc;
  switch (dtype) {
    case SF_F16: rc = launch_pack_v<__half>(a, stream); break;
    case SF_BF16: rc = launch_pack_v<__hip_bfloat16>(a, stream); break;
    default: rc = launch_pack_v<float>(a, stream); break;
  }
  timing_end(K_PACK, stream);
  return rc;
}

int launch_tiles(const TilesArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.ntiles + 3) / 4;
  if (blocks == 0) return (int)hipSuccess;
  const size_t lds = (a.ch_list != nullptr) ? (size_t)4 * a.c * sizeof(int32_t) : 0;
  timing_begin(K_TILES, stream);
  hipLaunchKernelGGL(k_tiles, dim3((unsigned)blocks), dim3(256), lds, stream, a);
  const int rc = (int)hipGetLastError();
  timing_end(K_TILES, stream);
  return rc;
}

}  // namespace sf

namespace sf {

int linear_words_per_row(int k) {
  const int w = (k + 31) / 32;
  return w <= 2 ? w : (w + 3) / 4 * 4;
}

int launch_pack_rows(const PackArgs& a, int dtype, hipStream_t stream) {
  const int64_t blocks = (a.total_chunks + 3) / 4;
  if (blocks == 0) return (int)hipSuccess;
  timing_begin(K_PACK_ROWS, stream);
  switch (dtype) {
    case SF_F16: hipLaunchKernelGGL(k_pack_rows<__half>, dim3((unsigned)blocks), dim3(256), 0, stream, a); break;
    case SF_BF16:
      hipLaunchKernelGGL(k_pack_rows<__hip_bfloat16>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
      break;
    default:
      if (a.c % 4 == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0)
        hipLaunchKernelGGL(k_pack_rows4, dim3((unsigned)blocks), dim3(256), 0, stream, a);
      else
        hipLaunchKernelGGL(k_pack_rows<float>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
      break;
  }
  timing_end(K_PACK_ROWS, stream);
  return (int)hipGetLastError();
}

}  // namespace sf
