// Device helpers shared by the row-tile Stage-2 kernels (3x3 and 1x1).
// gfx950 only.
#pragma once

#include "sf_internal.h"

namespace sf {

constexpr int kRowsWaves = 16;  // wavefronts per row-tile workgroup (one workgroup per CU)

// Number of compute units of the current device (cached per device).
int num_cus();

// Wavefronts per workgroup for a persistent kernel that runs one workgroup
// per CU over `wave_tiles` wave-sized tiles: as many passes as 16-wave
// workgroups would need, with the tiles spread evenly over them, so that no
// CU works through a last pass while the others idle.
inline int even_pass_waves(int64_t wave_tiles) {
  const int64_t cus = num_cus();
  const int64_t rounds = (wave_tiles + cus * kRowsWaves - 1) / (cus * kRowsWaves);
  const int64_t w = (wave_tiles + cus * rounds - 1) / (cus * rounds);
  return (int)(w < 1 ? 1 : (w > kRowsWaves ? kRowsWaves : w));
}

namespace {

// Exchange lane bit S with quad-slot bit S over v[4 * QP] (a butterfly stage
// of the register transpose).  Lanes with bit S set take the partner's upper
// slot; lanes with it clear take the partner's lower slot.
template <int S, int QP>
__device__ __forceinline__ void butterfly(float (&v)[4 * QP], int lane) {
#pragma unroll
  for (int j = 0; j < QP; ++j) {
    if (j & S) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ai = __float_as_int(v[4 * j + e]);
      const int bi = __float_as_int(v[4 * (j | S) + e]);
      int na, nb;
      if constexpr (S == 1 || S == 2) {
        constexpr int qp = S == 1 ? 0xB1 : 0x4E;  // quad_perm [1,0,3,2] / [2,3,0,1]
        const int pa = __builtin_amdgcn_mov_dpp(ai, qp, 0xf, 0xf, false);
        const int pb = __builtin_amdgcn_mov_dpp(bi, qp, 0xf, 0xf, false);
        const bool hi = (lane & S) != 0;
        na = hi ? pb : ai;
        nb = hi ? bi : pa;
      } else {
        // row_shl:S reads lane L+S, row_shr:S reads lane L-S; the bank mask
        // restricts each to the lanes whose bit S is clear / set.
        constexpr int shl = 0x100 | S, shr = 0x110 | S;
        constexpr int lo_banks = S == 4 ? 0x5 : 0x3, hi_banks = S == 4 ? 0xa : 0xc;
        nb = __builtin_amdgcn_update_dpp(bi, ai, shl, 0xf, lo_banks, false);
        na = __builtin_amdgcn_update_dpp(ai, bi, shr, 0xf, hi_banks, false);
      }
      v[4 * j + e] = __int_as_float(na);
      v[4 * (j | S) + e] = __int_as_float(nb);
    }
  }
}

template <typename T>
__device__ __forceinline__ void store4(T* p, float a, float b, float c, float d) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
  } else {
    const T h0 = from_f32<T>(a), h1 = from_f32<T>(b), h2 = from_f32<T>(c), h3 = from_f32<T>(d);
    uint16_t u0, u1, u2, u3;
    __builtin_memcpy(&u0, &h0, 2);
    __builtin_memcpy(&u1, &h1, 2);
    __builtin_memcpy(&u2, &h2, 2);
    __builtin_memcpy(&u3, &h3, 2);
    *reinterpret_cast<uint2*>(p) = make_uint2((uint32_t)u0 | ((uint32_t)u1 << 16), (uint32_t)u2 | ((uint32_t)u3 << 16));
  }
}

// Bitmap word type: both channel words of a pixel as one 64-bit value when
// the bitmap has two words per pixel.
template <int CWP> struct Word;
template <> struct Word<1> { typedef uint32_t type; };
template <> struct Word<2> { typedef uint64_t type; };

template <typename M>
__device__ __forceinline__ int lowest_bit(M m) {
  if constexpr (sizeof(M) == 8) return __builtin_ctzll(m);
  else return __builtin_ctz(m);
}

template <typename M>
__device__ __forceinline__ int pop_count(M m) {
  if constexpr (sizeof(M) == 8) return __builtin_popcountll(m);
  else return __builtin_popcount(m);
}

// ---------------------------------------------------------------------------
// Spike walk of a three-row window (3x3 stride-1 row kernels, lane = output
// channel, weight row (ci, kh, kw) of 64 channels at LDS byte offset
// (ci * 9 + kh * 3 + kw) * 256 from the lane's slot wlb).
//
// Positions are walked row by row (ia = 0, 1, 2), column by column (IB, a
// compile-time index), channels in ascending order.  Spike (ci, ia) at IB
// adds weight row (ci, kh = ia, kw) to acc[IB + D - kw] for each kw with
// 0 <= IB + D - kw < NACC (value tiles multiply it by xval(ci, ia, IB)), so
// every accumulator is a fixed register and receives its taps in the order
// (input row, input column, ci): deterministic, and the same in every kernel
// that walks this way.
//
// The walk runs on the scalar unit, whose issue rate (one instruction per
// SIMD every fourth cycle, shared by the SIMD's wavefronts) bounds it: per
// spike one find-first-set, a shift and xor that clear the bit and set the
// loop condition, and one multiply for the channel's row block; the row and
// tap offsets (kh * 768 + kw * 256) ride in the LDS instructions' immediate
// offsets.
// ---------------------------------------------------------------------------
template <int IA, int IB, int D, int NACC, bool VALUE, typename M, typename XV>
__device__ __forceinline__ void walk_position(float (&acc)[NACC], M m, const char* wlb, const XV& xval) {
  while (m) {
    const int ci = lowest_bit(m);
    m ^= (M)1 << ci;
    const char* base = wlb + ci * (9 * 256);
    float xv = 1.f;
    if constexpr (VALUE) xv = xval(ci, IA, IB);
#pragma unroll
    for (int kw = 0; kw < 3; ++kw) {
      const int o = IB + D - kw;
      if (o < 0 || o >= NACC) continue;
      const float wv = *reinterpret_cast<const float*>(base + (IA * 3 + kw) * 256);
      if constexpr (VALUE) acc[o] = fmaf(xv, wv, acc[o]);
      else acc[o] += wv;
    }
  }
}

template <int IA, int IB0, int U, int NB, int D, int NACC, bool VALUE, typename M, typename XV>
__device__ __forceinline__ void walk_batch(float (&acc)[NACC], const M (&mw)[NB], const char* wlb, const XV& xval) {
  if constexpr (U < NB) {
    walk_position<IA, IB0 + U, D, NACC, VALUE>(acc, mw[U], wlb, xval);
    walk_batch<IA, IB0, U + 1, NB, D, NACC, VALUE, M>(acc, mw, wlb, xval);
  }
}

// Positions (IA, IB .. NCOL - 1), words read eight at a time from
// word(ia, ib) (the channel word of window position (input row ia, column
// ib)) so that their scalar reads overlap.
template <int IA, int IB, int NCOL, int D, int NACC, bool VALUE, typename M, typename WF, typename XV>
__device__ __forceinline__ void walk_row(float (&acc)[NACC], const WF& word, const char* wlb, const XV& xval) {
  if constexpr (IB < NCOL) {
    constexpr int NB = (NCOL - IB) < 8 ? (NCOL - IB) : 8;
    M mw[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) mw[u] = word(IA, IB + u);
    walk_batch<IA, IB, 0, NB, D, NACC, VALUE, M>(acc, mw, wlb, xval);
    walk_row<IA, IB + NB, NCOL, D, NACC, VALUE, M>(acc, word, wlb, xval);
  }
}

// Rows IA .. 2 of the window; row 0 is skipped unless row0, row 2 unless
// row2 (rows outside the frame).
template <int IA, int NCOL, int D, int NACC, bool VALUE, typename M, typename WF, typename XV>
__device__ __forceinline__ void walk_window(float (&acc)[NACC], const WF& word, const char* wlb, const XV& xval,
                                            bool row0, bool row2) {
  if constexpr (IA < 3) {
    if ((IA != 0 || row0) && (IA != 2 || row2)) walk_row<IA, 0, NCOL, D, NACC, VALUE, M>(acc, word, wlb, xval);
    walk_window<IA + 1, NCOL, D, NACC, VALUE, M>(acc, word, wlb, xval, row0, row2);
  }
}

// Workgroup index as the tile loops see it.  The chip deals workgroups to
// its 8 XCDs round-robin (workgroup i runs on XCD i % 8), and each XCD has
// its own L2.  Remapping i -> (i % 8) * (n / 8) + i / 8 gives each XCD one
// contiguous range of the launch's (channel group, pass) work, so the
// bitmap words and weight chunks its workgroups share stay in its L2
// instead of every XCD touching every frame.  A bijection on [0, n) when
// n % 8 == 0 (the identity otherwise): placement changes speed, never
// results.
__device__ __forceinline__ int xcd_local_block(int i, int n) {
  constexpr int kXcds = 8;
  return (n % kXcds == 0) ? (i % kXcds) * (n / kXcds) + i / kXcds : i;
}

// xcd_local_block for any n: XCD x (workgroups i with i % 8 == x) takes the
// contiguous work range [x q + min(x, r), ...) of q + (x < r) items, q = n / 8,
// r = n % 8.  A bijection on [0, n).
__device__ __forceinline__ int xcd_range_block(int i, int n) {
  constexpr int kXcds = 8;
  const int q = n / kXcds, r = n % kXcds, x = i % kXcds;
  return x * q + min(x, r) + i / kXcds;
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(1))) void* gbl_ptr_t;

// OR of the non-binary chunk flags covering input rows ih_a .. ih_b (clamped
// to the frame).
__device__ __forceinline__ bool rows_value_path(const ConvArgs& a, const uint32_t* __restrict__ flags, int64_t frame,
                                                int ih_a, int ih_b) {
  ih_a = max(0, ih_a);
  ih_b = min(a.h_in - 1, ih_b);
  const int64_t c_a = ((int64_t)ih_a * a.w_in) / a.chunk;
  const int64_t c_b = ((int64_t)ih_b * a.w_in + a.w_in - 1) / a.chunk;
  const uint32_t* __restrict__ fl = flags + frame * a.chunks_per_frame;
  uint32_t f = 0u;
  for (int64_t q = c_a; q <= c_b; ++q) f |= fl[q];
  return f != 0u;
}

__device__ __forceinline__ float load_x(const void* __restrict__ x, int dtype, int64_t i) {
  if (dtype == SF_F16) return __half2float(static_cast<const __half*>(x)[i]);
  if (dtype == SF_BF16) return __bfloat162float(static_cast<const __hip_bfloat16*>(x)[i]);
  return static_cast<const float*>(x)[i];
}

// Store the tile (flattened run of npx pixels starting at run0) after the
// transpose: slot j of lane L holds channel (L & ~15) | j, pixels
// 4*(L & 15) .. +3 of the run.
template <typename TOut>
__device__ __forceinline__ void tile_store(float (&acc)[64], void* __restrict__ y, const ConvArgs& a, int64_t frame,
                                         int co0, int run0, int npx, int lane) {
  const int q = lane & 15, cb = lane & ~15;
  if (4 * q < npx) {
    TOut* yr = static_cast<TOut*>(y) + ((int64_t)frame * a.c_out + co0 + cb) * a.hw_out + run0 + 4 * q;
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (co0 + cb + j < a.c_out)
        store4<TOut>(yr + (int64_t)j * a.hw_out, acc[4 * j], acc[4 * j + 1], acc[4 * j + 2], acc[4 * j + 3]);
  }
}

// Multi-step LIF on the accumulators.  The membrane lives in the accumulator
// registers between steps, stored in the form that the next step's taps are
// added to:
//   decay_input:  acc = (tau - 1) V + V_r + b + sum  ->  H = acc / tau
//   otherwise:    acc = (1 - 1/tau) V + V_r / tau + b + sum  ->  H = acc
// (the same H as V + (I - (V - V_r)) / tau, resp. V - (V - V_r) / tau + I,
// with I = b + sum, up to rounding).
// Raw buffer access (gfx9 descriptor: 32-bit untyped, no swizzle): the
// per-lane byte offset sits in one VGPR and a uniform byte offset in an
// SGPR, so 64 channel planes of one pixel need no per-channel 64-bit
// addresses.  Offsets past num_records read 0 / drop the store.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)min(bytes, 0x7fffffffu), 0x00020000);
}
// Cache policy operand of the buffer stores: 0, or kStoreStream (the NT
// bit: the line is written through to HBM early instead of being kept for
// reuse).  Streaming pays for output written once in whole 128-byte lines;
// where a wavefront's run of a channel plane starts inside a line, the
// neighbouring run's half arrives after the line has left, and the line is
// written twice (measured slower at 28 x 28 and 14 x 14 planes).
constexpr int kStoreStream = 2;

template <typename T>
struct BufIO;
template <>
struct BufIO<float> {
  static __device__ __forceinline__ float load(__amdgpu_buffer_rsrc_t r, int vo, int so) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0));
  }
  template <int CP = 0>
  static __device__ __forceinline__ void store(float v, __amdgpu_buffer_rsrc_t r, int vo, int so) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, v), r, vo, so, CP);
  }
};
template <>
struct BufIO<__half> {
  static __device__ __forceinline__ __half load(__amdgpu_buffer_rsrc_t r, int vo, int so) {
    return __builtin_bit_cast(__half, __builtin_amdgcn_raw_buffer_load_b16(r, vo, so, 0));
  }
  template <int CP = 0>
  static __device__ __forceinline__ void store(__half v, __amdgpu_buffer_rsrc_t r, int vo, int so) {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), r, vo, so, CP);
  }
};
template <>
struct BufIO<__hip_bfloat16> {
  static __device__ __forceinline__ __hip_bfloat16 load(__amdgpu_buffer_rsrc_t r, int vo, int so) {
    return __builtin_bit_cast(__hip_bfloat16, __builtin_amdgcn_raw_buffer_load_b16(r, vo, so, 0));
  }
  template <int CP = 0>
  static __device__ __forceinline__ void store(__hip_bfloat16 v, __amdgpu_buffer_rsrc_t r, int vo, int so) {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), r, vo, so, CP);
  }
};

// Bitmap word c of each of a lane's nine 3x3 input taps (stride / padding of
// a, top-left tap at (ih0, iw0); 0 outside the frame), through one buffer
// resource over every frame's bitmap (below 2^31 bytes) with the frame's
// start as the per-lane byte offset fbase.  Word c of pixel q sits at
// q * bm_ps + c * bm_ws words from the frame's start (pixel-major words or
// word planes).  A tap outside the frame gets an offset past num_records,
// which the hardware returns as 0.
__device__ __forceinline__ void px3_load_words_at(uint32_t (&w)[9], __amdgpu_buffer_rsrc_t rs, uint32_t fbase,
                                                  const ConvArgs& a, int ih0, int iw0, int c) {
  const uint32_t cofs = (uint32_t)c * (uint32_t)a.bm_ws;
#pragma unroll
  for (int tp = 0; tp < 9; ++tp) {
    const int ih = ih0 + tp / 3, iw = iw0 + tp % 3;
    const bool in = ih >= 0 && ih < a.h_in && iw >= 0 && iw < a.w_in;
    const uint32_t off = in ? fbase + ((uint32_t)(ih * a.w_in + iw) * (uint32_t)a.bm_ps + cofs) * 4u : 0x80000000u;
    w[tp] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)off, 0, 0);
  }
}

// Four consecutive 0/1 values (bits 0..3 of q) as one 16-byte (f32) or
// 8-byte (f16 / bf16) buffer store.  The whole offset goes in the VGPR and
// soffset is the constant 0: with an SGPR soffset the compiler adds no wait
// state between a 16-byte store and a VALU write of its data registers, and
// on gfx950 the last lanes of each 16-lane group then store the overwritten
// value.  Spikes are written once, with the streaming policy (the fused
// conv-LIF forwards measured faster with it).
typedef unsigned int sf_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int sf_u32x2 __attribute__((ext_vector_type(2)));
template <typename T>
__device__ __forceinline__ void store_bits4(uint32_t q, __amdgpu_buffer_rsrc_t r, int vo) {
  asm volatile("" : "+v"(vo));  // keep the offset in the VGPR operand
  constexpr int so = 0;
  if constexpr (sizeof(T) == 4) {
    constexpr uint32_t one = 0x3f800000u;  // 1.0f
    const sf_u32x4 v = {(q & 1u) ? one : 0u, (q & 2u) ? one : 0u, (q & 4u) ? one : 0u, (q & 8u) ? one : 0u};
    __builtin_amdgcn_raw_buffer_store_b128(v, r, vo, so, kStoreStream);
  } else {
    constexpr uint32_t one = std::is_same<T, __half>::value ? 0x3c00u : 0x3f80u;  // 1.0 in f16 / bf16
    const sf_u32x2 v = {((q & 1u) ? one : 0u) | ((q & 2u) ? one << 16 : 0u),
                        ((q & 4u) ? one : 0u) | ((q & 8u) ? one << 16 : 0u)};
    __builtin_amdgcn_raw_buffer_store_b64(v, r, vo, so, kStoreStream);
  }
}

// The LIF charge step in the accumulators: with acc = a * V + vr_term + I,
//   decay_input:  H = V + (I - (V - Vr)) / tau = acc / tau  (a = tau - 1, vr_term = Vr)
//   otherwise:    H = V - (V - Vr) / tau + I  = acc        (a = 1 - 1/tau, vr_term = Vr / tau)
// (Vr = v_reset for hard reset, 0 for soft reset), so the current I (bias +
// spike sums + residual) is accumulated on top of the seeded membrane.
struct LifCoef {
  float a, vr_term, inv_tau, v_th, v_reset;
  bool hard, decay_input;
};

// Seed from per-channel constants staged in LDS (vr_term + bias): LDS
// reads do not queue behind the wave's outstanding global stores.
template <int CO>
__device__ __forceinline__ void lif_seed_lds(float (&acc)[CO], const LifCoef& L, const float* seed) {
#pragma unroll
  for (int co = 0; co < CO; ++co) acc[co] = fmaf(L.a, acc[co], seed[co]);
}

// LIF coefficients from the launch arguments.
__device__ __forceinline__ LifCoef lif_coef(const ConvArgs& a) {
  LifCoef L;
  L.inv_tau = 1.f / a.tau;
  L.decay_input = a.decay_input != 0;
  L.hard = a.hard_reset != 0;
  L.v_th = a.v_th;
  L.v_reset = a.v_reset;
  const float vr = L.hard ? a.v_reset : 0.f;
  L.a = L.decay_input ? a.tau - 1.f : 1.f - L.inv_tau;
  L.vr_term = L.decay_input ? vr : vr * L.inv_tau;
  return L;
}

}  // namespace

}  // namespace sf
