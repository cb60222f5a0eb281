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

// Stores a wavefront's 64 x 64 accumulator tile (acc[rt][ct] element i of
// lane l: row 16 rt + 4 (l >> 4) + i, column 16 ct + (l & 15)) plus the bias
// as rows of 16-byte pieces: each 16-row slice goes through the wavefront's
// own LDS region (16 rows of 68 floats: conflict-free both ways) and is read
// back as four consecutive columns per lane, so that one store instruction
// writes four 256-byte row runs (4-byte stores scattered over the rows
// wrote y at ~1.4 TB/s).  r_0, c_0: the tile's first row and column in y.
template <typename TOut>
__device__ __forceinline__ void lm_store_tile(const f32x4 (&acc)[4][4], float* __restrict__ stile,
                                              const float* __restrict__ bias, TOut* __restrict__ Y, int64_t m,
                                              int c_out, int64_t r_0, int c_0, int lane) {
  constexpr int kS = 68;  // floats per staged row
  const int g = lane >> 4, li = lane & 15;
  float bv[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const int col = c_0 + 16 * ct + li;
    bv[ct] = bias != nullptr && col < c_out ? bias[col] : 0.f;
  }
  const int rq = lane >> 4, cq = 4 * (lane & 15);  // read-back: rows rq + 4 j, columns cq .. cq + 3
  const int col = c_0 + cq;
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i) stile[(4 * g + i) * kS + 16 * ct + li] = acc[rt][ct][i] + bv[ct];
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wavefront's writes are done before its reads
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t row = r_0 + 16 * rt + rq + 4 * j;
      const float4 v = *reinterpret_cast<const float4*>(&stile[(rq + 4 * j) * kS + cq]);
      if (row < m && col < c_out) store4<TOut>(Y + row * c_out + col, v.x, v.y, v.z, v.w);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // its reads are done before the next slice's writes
  }
}

template <typename TIn, typename TOut, bool VEC>
__global__ __launch_bounds__(256) void k_linear_mfma(LinMfmaArgs a) {
  // Double-buffered LDS tiles (bf16 bit patterns): x [128 rows][32] (its hi
  // part in the main walk, its lo part in the second), W hi / lo [128
  // columns][32]; 48 KB, in one array (the output staging reuses it).
  __shared__ __align__(16) uint16_t s_tiles[3][2][kLmRows * kLmLda];
  auto& s_xh = s_tiles[0];
  auto& s_wh = s_tiles[1];
  auto& s_wl = s_tiles[2];
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

  // The last step's barrier: every wavefront is done with the tiles.
  float* stile = reinterpret_cast<float*>(&s_tiles[0][0][0]) + wave * (16 * 68);
  lm_store_tile<TOut>(acc, stile, a.bias, static_cast<TOut*>(a.y), a.m, a.c_out, r0 + 64 * wr, c0 + 64 * wc, lane);
}

// ---- the same product over the prescan's row bitmap --------------------
//
// For spike inputs the x tile is one bit per element: a lane's A fragment
// (8 consecutive k of one row) is one byte of that row's bitmap word, its
// bits turned into bf16 0 / 1 values on the VALU, so x costs 4 bytes per row
// per 32-wide K step instead of 128 (f32) and needs no staging.  A
// workgroup of 4 wavefronts computes one 256 x 128 tile, each wavefront
// 128 x 64 (8 x 4 MFMA tiles: a step's 8 W fragment reads serve 64
// products); per step the W tiles (bf16 hi and lo, 16 KB) and the rows'
// bitmap words (1 KB) go from global memory straight into a ring of three
// LDS buffers, requested two steps ahead and waited for by count.
// The barrier that ends a step waits for no load (in-kernel timestamps of a
// __syncthreads() version showed every step waiting for all of them), and
// 66.5 KB of LDS let two workgroups share a CU: their barriers are
// independent, so one's fragment reads and waits overlap the other's
// MFMAs, and a finished workgroup's stores drain while the next one on the
// CU starts (a persistent version with one 8-wavefront workgroup per CU
// stored every tile in lockstep on all CUs, ~6 us a round with the matrix
// cores idle).  Row blocks whose non-binary flag is set (a value other than 0 and
// 1 in some row) read their x tiles instead: A fragments from x split into
// bf16 hi + lo, three products per step (the exactness of the direct
// kernel).
// Barrier for LDS hand-offs: this wavefront's LDS accesses are complete
// before it, and the compiler moves no memory access across it.  Unlike
// __syncthreads() (whose release fence waits for every outstanding load,
// the direct LDS loads included) it leaves the loads of later steps in
// flight; their consumers wait for them by count.
__device__ __forceinline__ void ws_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

constexpr int kLbRows = 256;    // rows per workgroup tile
constexpr int kLbWaves = 4;
constexpr int kLbRT = 8;        // 16-row MFMA tiles per wavefront (128 rows)
constexpr int kLbBufs = 3;      // stage buffers (W tiles and words of one 32-wide K step)

// W tiles of step s (both parts) into LDS buffers (sh, sl) with direct
// loads: 1 KB blocks, wavefront w loading blocks 4 w .. 4 w + 3 (blocks 0..7
// the hi part, 8..15 the lo part); LDS position q of a part holds row q >> 2,
// stored piece q & 3, i.e. logical piece lm_piece(row, q & 3) (lm_piece is
// its own inverse).  Rows past c_out load row 0 (never stored).
__device__ __forceinline__ void lb_load_w(uint16_t* __restrict__ sh, uint16_t* __restrict__ sl,
                                          const uint16_t* __restrict__ wh, const uint16_t* __restrict__ wl, int kp,
                                          int c0, int c_out, int s, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < 16 / kLbWaves; ++j) {
    const int u = (16 / kLbWaves) * wave + j;
    const int q = (u & 7) * 64 + lane;
    const int r = q >> 2;
    const int p = lm_piece(r, q & 3);
    const int col = c0 + r < c_out ? c0 + r : 0;
    const uint16_t* src = (u < 8 ? wh : wl) + (int64_t)col * kp + 32 * s + 8 * p;
    uint16_t* dst = (u < 8 ? sh : sl) + (u & 7) * 512;  // 1 KB = 512 bf16
    __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)dst, 16, 0, 0);
  }
}
constexpr int kLbLoads = 16 / kLbWaves + 1;  // direct loads per wavefront and step (W blocks, words)

// Eight spikes (bits 0..7 of byte) as bf16 0 / 1 values, element i = bit i.
__device__ __forceinline__ bf16x8 spike_bf16x8(uint32_t byte) {
  uint32_t p[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    p[j] = (((byte >> (2 * j)) & 1u) * 0x3F80u) | (((byte >> (2 * j + 1)) & 1u) * 0x3F800000u);
  return __builtin_bit_cast(bf16x8, make_uint4(p[0], p[1], p[2], p[3]));
}

// A wavefront's (16 RT) x 64 tile as rows of 16-byte pieces (lm_store_tile's
// staging) through buffer stores: rows past m and columns past c_out fall
// outside the buffer range and are dropped.  The whole offset rides in the
// VGPR, soffset stays 0 (with an SGPR soffset the compiler adds no wait
// state between a 16-byte store and a VALU write of its data registers, and
// on gfx950 the last lanes of each 16-lane group then store the overwritten
// value).
template <int RT, typename TOut>
__device__ __forceinline__ void lb_store_tile(const f32x4 (&acc)[RT][4], float* __restrict__ stile,
                                              const float* __restrict__ bias, __amdgpu_buffer_rsrc_t ry, int64_t m,
                                              int c_out, int64_t r_0, int c_0, int lane) {
  constexpr int kS = 68;
  const int g = lane >> 4, li = lane & 15;
  float bv[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const int col = c_0 + 16 * ct + li;
    bv[ct] = bias != nullptr && col < c_out ? bias[col] : 0.f;
  }
  const int rq = lane >> 4, cq = 4 * (lane & 15);
  const int col = c_0 + cq;
  constexpr uint32_t B = (uint32_t)sizeof(TOut);
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i) stile[(4 * g + i) * kS + 16 * ct + li] = acc[rt][ct][i] + bv[ct];
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t row = r_0 + 16 * rt + rq + 4 * j;
      const float4 v = *reinterpret_cast<const float4*>(&stile[(rq + 4 * j) * kS + cq]);
      int vo = (row < m && col < c_out) ? (int)((uint32_t)(row * c_out + col) * B) : 0x7fffffff;
      asm volatile("" : "+v"(vo));
      if constexpr (sizeof(TOut) == 4) {
        const sf_u32x4 q = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
        __builtin_amdgcn_raw_buffer_store_b128(q, ry, vo, 0, 0);
      } else {
        const TOut h0 = from_f32<TOut>(v.x), h1 = from_f32<TOut>(v.y), h2 = from_f32<TOut>(v.z), h3 = from_f32<TOut>(v.w);
        const sf_u32x2 q = {(uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16),
                            (uint32_t)__builtin_bit_cast(uint16_t, h2) | ((uint32_t)__builtin_bit_cast(uint16_t, h3) << 16)};
        __builtin_amdgcn_raw_buffer_store_b64(q, ry, vo, 0, 0);
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
}

// One workgroup per 256 x 128 tile (placed XCD-locally: the column blocks
// of a row block run on one XCD and share its rows' words through L2).
template <typename TIn, typename TOut>
__global__ __launch_bounds__(64 * kLbWaves, 2) void k_linear_bits_mfma(LinMfmaArgs a, const uint32_t* __restrict__ bits,
                                                                    const uint32_t* __restrict__ flags, int cwp) {
  __shared__ __align__(16) uint16_t s_wh[kLbBufs][kLmCols * kLmLda];
  __shared__ __align__(16) uint16_t s_wl[kLbBufs][kLmCols * kLmLda];
  __shared__ __align__(16) uint32_t s_words[kLbBufs][kLbRows];  // bitmap word of each row, per step
  __shared__ __align__(16) float s_out[kLbWaves * 16 * 68];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wr = wave >> 1, wc = wave & 1;
  const int g = lane >> 4, li = lane & 15;
  const int ncb = (a.c_out + kLmCols - 1) / kLmCols;
  const int nsteps = a.kp / kLmK;
  const int64_t nchunks = (a.m + kLinearRowChunk - 1) / kLinearRowChunk;
  const int bid = xcd_range_block((int)blockIdx.x, (int)gridDim.x);
  const int64_t rb = bid / ncb;
  const int64_t r0 = rb * kLbRows;
  const int c0 = (int)(bid - rb * ncb) * kLmCols;
  const TIn* __restrict__ X = static_cast<const TIn*>(a.x);

  // Step t's bitmap words for the tile's 256 rows (wavefront w: LDS
  // positions 64 w .. 64 w + 63, one word per lane).  Position q holds tile
  // row 128 (q >> 7) + 16 (q & 7) + ((q >> 3) & 15): the words of a lane's
  // eight row tiles (lane li of wavefront row wr: rows 128 wr + 16 rt + li)
  // are consecutive, two 16-byte reads.  Rows past m load row 0's word:
  // their outputs are never stored.
  auto load_step = [&](int t) {
    const int b = t % kLbBufs;
    lb_load_w(s_wh[b], s_wl[b], a.wh, a.wl, a.kp, c0, a.c_out, t, wave, lane);
    const int q = 64 * wave + lane;
    const int64_t row = r0 + 128 * (q >> 7) + 16 * (q & 7) + ((q >> 3) & 15);
    const uint32_t* src = bits + (row < a.m ? row : 0) * (int64_t)cwp + t;
    __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)&s_words[b][64 * wave], 4, 0, 0);
  };
  auto bfrags = [&](int b, bf16x8 (&bh)[4], bf16x8 (&bl)[4]) {
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int r = 64 * wc + 16 * ct + li;
      const int c = r * kLmLda + 8 * lm_piece(r, g);
      bh[ct] = *reinterpret_cast<const bf16x8*>(&s_wh[b][c]);
      bl[ct] = *reinterpret_cast<const bf16x8*>(&s_wl[b][c]);
    }
  };
  // Every global load of the spike path is a direct LDS load, waited for by
  // count (the compiler would wait for all of them before the first use of
  // any register load): steps 0 and 1 first, step 0's are waited for.
  load_step(0);
  if (nsteps > 1) load_step(1);
  if (nsteps > 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLbLoads) : "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // The row block's non-binary flags (one per 16 rows, read by every
  // wavefront with uniform loads) decide its A operand.
  uint32_t fl = 0u;
  const int64_t ch0 = r0 / kLinearRowChunk;
#pragma unroll
  for (int i = 0; i < kLbRows / kLinearRowChunk; ++i)
    if (ch0 + i < nchunks) fl |= flags[ch0 + i];
  const bool value = fl != 0u;
  ws_barrier();  // step 0's tiles of every wavefront

  f32x4 acc[kLbRT][4];
#pragma unroll
  for (int i = 0; i < kLbRT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (!value) {
    for (int s = 0; s < nsteps; ++s) {
      const int b = s % kLbBufs;
      // A fragments: byte g of each row tile's word, its 8 bits turned into
      // bf16 0 / 1 on the VALU; B fragments from the W tiles.
      const uint4 w0 = *reinterpret_cast<const uint4*>(&s_words[b][8 * (16 * wr + li)]);
      const uint4 w1 = *reinterpret_cast<const uint4*>(&s_words[b][8 * (16 * wr + li) + 4]);
      const uint32_t wd[kLbRT] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      bf16x8 af[kLbRT];
#pragma unroll
      for (int rt = 0; rt < kLbRT; ++rt) af[rt] = spike_bf16x8(__builtin_amdgcn_ubfe(wd[rt], 8 * g, 8));
      bf16x8 bh[4], bl[4];
      bfrags(b, bh, bl);
#pragma unroll
      for (int rt = 0; rt < kLbRT; ++rt)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
          acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[rt], bh[ct], acc[rt][ct], 0, 0, 0);
#pragma unroll
      for (int rt = 0; rt < kLbRT; ++rt)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
          acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[rt], bl[ct], acc[rt][ct], 0, 0, 0);
      // Step s + 2's loads, behind the MFMAs (its buffer was last read by
      // step s - 1, before the previous barrier); then step s + 1's have
      // landed (only the ones just issued may still be in flight).
      if (s + 2 < nsteps) {
        load_step(s + 2);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLbLoads) : "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      ws_barrier();
    }
  } else {
    // x tiles: lane (li, g) reads k = 32 s + 8 g .. + 7 of its rows; past k
    // and past m the elements are 0; |x| < cutoff counts as 0.  The eight
    // row tiles in two halves (registers).
    const bool vec4 = sizeof(TIn) == 4 && (a.k & 3) == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0;
    for (int s = 0; s < nsteps; ++s) {
      if (s + 2 < nsteps) load_step(s + 2);  // its buffer was last read by step s - 1
      bf16x8 bh[4], bl[4];
      bfrags(s % kLbBufs, bh, bl);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
      bf16x8 ah[4], al[4];
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const int64_t row = r0 + 128 * wr + 16 * (4 * half + rt) + li;
        const int kk0 = 32 * s + 8 * g;
        float v8[8];
        if (vec4) {
          // f32 rows, k % 4 == 0, 16-byte aligned: two 16-byte loads, each
          // wholly inside or past the row.
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const bool ok = row < a.m && kk0 + 4 * h < a.k;
            const float4 t = *reinterpret_cast<const float4*>(ok ? reinterpret_cast<const float*>(X) + row * a.k + kk0 + 4 * h
                                                                 : reinterpret_cast<const float*>(X));
            v8[4 * h] = ok ? t.x : 0.f;
            v8[4 * h + 1] = ok ? t.y : 0.f;
            v8[4 * h + 2] = ok ? t.z : 0.f;
            v8[4 * h + 3] = ok ? t.w : 0.f;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int kk = kk0 + e;
            v8[e] = (row < a.m && kk < a.k) ? to_f32<TIn>(X[row * a.k + kk]) : 0.f;
          }
        }
        uint32_t hx[4], lx[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float v2[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) v2[e] = fabsf(v8[2 * j + e]) >= a.cutoff ? v8[2 * j + e] : 0.f;
          const uint16_t h0 = bf16_bits(v2[0]), h1 = bf16_bits(v2[1]);
          hx[j] = (uint32_t)h0 | ((uint32_t)h1 << 16);
          lx[j] = (uint32_t)bf16_bits(v2[0] - bf16_value(h0)) | ((uint32_t)bf16_bits(v2[1] - bf16_value(h1)) << 16);
        }
        ah[rt] = __builtin_bit_cast(bf16x8, make_uint4(hx[0], hx[1], hx[2], hx[3]));
        al[rt] = __builtin_bit_cast(bf16x8, make_uint4(lx[0], lx[1], lx[2], lx[3]));
      }
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          f32x4& c = acc[4 * half + rt][ct];
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[rt], bh[ct], c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[rt], bl[ct], c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[rt], bh[ct], c, 0, 0, 0);
        }
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);  // the tiles of step s + 1 (the x loads are waited for already)
      __syncthreads();
    }
  }
  // The last step's barrier: every wavefront is done with the buffers.
  const auto rs_y = buf_rsrc(a.y, (uint32_t)((uint64_t)a.m * (uint64_t)a.c_out * sizeof(TOut)));
  lb_store_tile<kLbRT, TOut>(acc, &s_out[wave * 16 * 68], a.bias, rs_y, a.m, a.c_out, r0 + 128 * wr, c0 + 64 * wc,
                             lane);
}

template <typename TIn>
int launch_lb_d(const LinMfmaArgs& a, const uint32_t* bits, const uint32_t* flags, int cwp, int out_dtype,
                hipStream_t stream) {
  const int64_t tiles = ((a.m + kLbRows - 1) / kLbRows) * ((a.c_out + kLmCols - 1) / kLmCols);
  if (tiles == 0) return (int)hipSuccess;
  if (out_dtype == SF_F32)
    hipLaunchKernelGGL((k_linear_bits_mfma<TIn, float>), dim3((unsigned)tiles), dim3(64 * kLbWaves), 0, stream, a,
                       bits, flags, cwp);
  else
    hipLaunchKernelGGL((k_linear_bits_mfma<TIn, TIn>), dim3((unsigned)tiles), dim3(64 * kLbWaves), 0, stream, a, bits,
                       flags, cwp);
  return (int)hipGetLastError();
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

int launch_linear_bits_mfma(const LinMfmaArgs& a, const uint32_t* bits, const uint32_t* flags, int cwp, int in_dtype,
                            int out_dtype, hipStream_t stream) {
  timing_begin(K_LINEAR_MFMA, stream);
  const int rc = in_dtype == SF_F16    ? launch_lb_d<__half>(a, bits, flags, cwp, out_dtype, stream)
                 : in_dtype == SF_BF16 ? launch_lb_d<__hip_bfloat16>(a, bits, flags, cwp, out_dtype, stream)
                                       : launch_lb_d<float>(a, bits, flags, cwp, out_dtype, stream);
  timing_end(K_LINEAR_MFMA, stream);
  return rc;
}

int launch_linear_mfma(const LinMfmaArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  timing_begin(K_LINEAR_MFMA, stream);
  const int rc = in_dtype == SF_F16    ? launch_lm_d<__half>(a, out_dtype, stream)
                 : in_dtype == SF_BF16 ? launch_lm_d<__hip_bfloat16>(a, out_dtype, stream)
                                       : launch_lm_d<float>(a, out_dtype, stream);
  timing_end(K_LINEAR_MFMA, stream);
  return rc;
}

}  // namespace sf
