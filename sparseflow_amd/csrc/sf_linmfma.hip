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
// (8 consecutive k of one row) is one byte of that row's bitmap word, turned
// into bf16 0 / 1 values by a 16-entry nibble table, so x costs 4 bytes per
// row per 32-wide K step instead of 128 (f32) and needs no staging.  One
// workgroup of 8 wavefronts computes a 256-row x 128-column tile (each
// wavefront 64 x 64 as above); per step only the W tiles (bf16 hi and lo,
// 16 KB) are staged, with direct global->LDS loads two steps ahead into
// three LDS buffers, and each lane's bitmap words two steps ahead in
// registers.  Row blocks whose non-binary flag is set (a value other than 0
// and 1 in some row) read their x tiles instead: A fragments from x split
// into bf16 hi + lo, three products per step (the exactness of the direct
// kernel).
constexpr int kLbRows = 256;    // rows per workgroup tile
constexpr int kLbWaves = 8;
constexpr int kLbBufs = 3;      // W stage buffers

// W tiles of step s (both parts) into LDS buffer b with direct loads: 1 KB
// blocks, wavefront w loading blocks 2 w and 2 w + 1 (blocks 0..7 the hi part,
// 8..15 the lo part); LDS position q of a part holds row q >> 2, stored piece
// q & 3, i.e. logical piece (q & 3) ^ ((row >> 1) & 3) (lm_piece is its own
// inverse).  Rows past c_out load row 0 (never stored).
__device__ __forceinline__ void lb_load_w(uint16_t* __restrict__ sh, uint16_t* __restrict__ sl,
                                          const uint16_t* __restrict__ wh, const uint16_t* __restrict__ wl, int kp,
                                          int c0, int c_out, int s, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int u = 2 * wave + j;
    const int q = (u & 7) * 64 + lane;
    const int r = q >> 2;
    const int p = lm_piece(r, q & 3);
    const int col = c0 + r < c_out ? c0 + r : 0;
    const uint16_t* src = (u < 8 ? wh : wl) + (int64_t)col * kp + 32 * s + 8 * p;
    uint16_t* dst = (u < 8 ? sh : sl) + (u & 7) * 512;  // 1 KB = 512 bf16
    __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)dst, 16, 0, 0);
  }
}

// A wavefront's 64 x 64 tile as rows of 16-byte pieces (lm_store_tile's
// staging) through buffer stores: every lane issues exactly 16 stores (rows
// past m and columns past c_out fall outside the buffer range and are
// dropped), so a following wait for loads issued before them can name its
// count.  The whole offset rides in the VGPR, soffset stays 0 (with an SGPR
// soffset the compiler adds no wait state between a 16-byte store and a
// VALU write of its data registers, and on gfx950 the last lanes of each
// 16-lane group then store the overwritten value).
template <typename TOut>
__device__ __forceinline__ void lb_store_tile(const f32x4 (&acc)[4][4], float* __restrict__ stile,
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
  for (int rt = 0; rt < 4; ++rt) {
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

// Persistent: workgroup i takes tiles i, i + grid, ... (the grid a multiple
// of 8, so a tile runs on XCD tile % 8 and xcd_range_block keeps a row
// block's column tiles on one XCD).  The next tile's first W tiles and
// bitmap words are requested before this tile's output is stored, so the
// stores drain while the next tile starts.
template <typename TIn, typename TOut>
__global__ __launch_bounds__(64 * kLbWaves) void k_linear_bits_mfma(LinMfmaArgs a, const uint32_t* __restrict__ bits,
                                                                    const uint32_t* __restrict__ flags, int cwp) {
  // W hi tiles (buffers 0..2), then W lo tiles; the output staging (16 rows
  // of 68 floats per wavefront) apart, so that the next tile's loads may
  // land while this one's output is staged.
  __shared__ __align__(16) uint16_t s_wbuf[2 * kLbBufs * kLmCols * kLmLda];
  __shared__ __align__(16) float s_out[kLbWaves * 16 * 68];
  __shared__ __align__(16) uint2 s_tab[16];
  uint16_t (*s_wh)[kLmCols * kLmLda] = reinterpret_cast<uint16_t (*)[kLmCols * kLmLda]>(&s_wbuf[0]);
  uint16_t (*s_wl)[kLmCols * kLmLda] = reinterpret_cast<uint16_t (*)[kLmCols * kLmLda]>(&s_wbuf[kLbBufs * kLmCols * kLmLda]);
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave >> 1, wc = wave & 1;
  const int g = lane >> 4, li = lane & 15;
  const int ncb = (a.c_out + kLmCols - 1) / kLmCols;
  const int64_t ntiles = ((a.m + kLbRows - 1) / kLbRows) * ncb;
  const int nsteps = a.kp / kLmK;
  const int64_t nchunks = (a.m + kLinearRowChunk - 1) / kLinearRowChunk;
  if (tid < 16) {
    const uint32_t b = (uint32_t)tid;
    s_tab[tid] = make_uint2(((b & 1u) ? 0x3F80u : 0u) | ((b & 2u) ? 0x3F800000u : 0u),
                            ((b & 4u) ? 0x3F80u : 0u) | ((b & 8u) ? 0x3F800000u : 0u));
  }
  const auto rs_b = buf_rsrc(bits, (uint32_t)((uint64_t)a.m * (uint64_t)cwp * 4u));
  const auto rs_y = buf_rsrc(a.y, (uint32_t)((uint64_t)a.m * (uint64_t)a.c_out * sizeof(TOut)));
  float* stile = &s_out[wave * 16 * 68];
  const TIn* __restrict__ X = static_cast<const TIn*>(a.x);

  int64_t r0 = 0;
  int c0 = 0;
  uint32_t rowoff[4];
  auto place = [&](int64_t tile) {
    const int bid = xcd_range_block((int)tile, (int)ntiles);
    const int64_t rb = bid / ncb;
    r0 = rb * kLbRows;
    c0 = (int)(bid - rb * ncb) * kLmCols;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) rowoff[rt] = (uint32_t)(r0 + 64 * wr + 16 * rt + li) * (uint32_t)cwp * 4u;
  };
  auto load_words = [&](uint32_t (&w)[4], int s) {
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) w[rt] = __builtin_amdgcn_raw_buffer_load_b32(rs_b, (int)(rowoff[rt] + 4u * s), 0, 0);
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
  // A tile's first loads: W tiles of steps 0 and 1 (2 + 2 per lane) and the
  // words of steps 0 and 1 (4 + 4).
  uint32_t wa[4], wb[4];
  auto first_loads = [&]() {
    lb_load_w(s_wh[0], s_wl[0], a.wh, a.wl, a.kp, c0, a.c_out, 0, wave, lane);
    if (nsteps > 1) lb_load_w(s_wh[1], s_wl[1], a.wh, a.wl, a.kp, c0, a.c_out, 1, wave, lane);
    load_words(wa, 0);
    if (nsteps > 1) load_words(wb, 1);
  };

  int64_t tile = blockIdx.x;
  if (tile < ntiles) {
    place(tile);
    first_loads();
  }
  bool first = true;
  for (; tile < ntiles; tile += gridDim.x) {
    // The first loads of this tile have landed (the previous tile's 16
    // stores per lane were issued after them); the barrier publishes the W
    // tiles (and, on the first tile, the table).  The row block's
    // non-binary flags (one per 16 rows) decide its A operand.
    if (first) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    else __builtin_amdgcn_s_waitcnt(0x4F70);        // vmcnt(16)
    first = false;
    const int64_t ch = r0 / kLinearRowChunk + tid;
    const bool value = __syncthreads_or(tid < kLbRows / kLinearRowChunk && ch < nchunks && flags[ch] != 0u) != 0;
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Before the barrier that ends step s: the W tiles of step s + 1 have
    // landed (the only loads issued after them are those of step s + 2, at
    // most 2 + 4 per lane, and the words of step s + 1, 4).
    auto wait_next_w = [&](int s) {
      if (s + 2 < nsteps) __builtin_amdgcn_s_waitcnt(0x0F7A);  // vmcnt(10)
      else __builtin_amdgcn_s_waitcnt(0x0F70);                 // vmcnt(0)
    };
    if (!value) {
      auto step = [&](int s, uint32_t (&w)[4]) {
        if (s + 2 < nsteps)
          lb_load_w(s_wh[(s + 2) % kLbBufs], s_wl[(s + 2) % kLbBufs], a.wh, a.wl, a.kp, c0, a.c_out, s + 2, wave, lane);
        bf16x8 af[4];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
          const uint32_t byte = __builtin_amdgcn_ubfe(w[rt], 8 * g, 8);
          const uint2 lo = s_tab[byte & 15u], hi = s_tab[byte >> 4];
          af[rt] = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
        }
        if (s + 2 < nsteps) load_words(w, s + 2);
        bf16x8 bh[4], bl[4];
        bfrags(s % kLbBufs, bh, bl);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
          for (int ct = 0; ct < 4; ++ct)
            acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[rt], bh[ct], acc[rt][ct], 0, 0, 0);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
          for (int ct = 0; ct < 4; ++ct)
            acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[rt], bl[ct], acc[rt][ct], 0, 0, 0);
        wait_next_w(s);
        __syncthreads();
      };
      for (int s = 0; s < nsteps; s += 2) {
        step(s, wa);
        if (s + 1 < nsteps) step(s + 1, wb);
      }
    } else {
      // x tiles: lane (li, g) reads k = 32 s + 8 g .. + 7 of its rows; past
      // k and past m the elements are 0; |x| < cutoff counts as 0.
      for (int s = 0; s < nsteps; ++s) {
        if (s + 2 < nsteps)
          lb_load_w(s_wh[(s + 2) % kLbBufs], s_wl[(s + 2) % kLbBufs], a.wh, a.wl, a.kp, c0, a.c_out, s + 2, wave, lane);
        bf16x8 ah[4], al[4];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
          const int64_t row = r0 + 64 * wr + 16 * rt + li;
          const int kk0 = 32 * s + 8 * g;
          uint32_t hx[4], lx[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float v2[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const int kk = kk0 + 2 * j + e;
              const float t = (row < a.m && kk < a.k) ? to_f32<TIn>(X[row * a.k + kk]) : 0.f;
              v2[e] = fabsf(t) >= a.cutoff ? t : 0.f;
            }
            const uint16_t h0 = bf16_bits(v2[0]), h1 = bf16_bits(v2[1]);
            hx[j] = (uint32_t)h0 | ((uint32_t)h1 << 16);
            lx[j] = (uint32_t)bf16_bits(v2[0] - bf16_value(h0)) | ((uint32_t)bf16_bits(v2[1] - bf16_value(h1)) << 16);
          }
          ah[rt] = __builtin_bit_cast(bf16x8, make_uint4(hx[0], hx[1], hx[2], hx[3]));
          al[rt] = __builtin_bit_cast(bf16x8, make_uint4(lx[0], lx[1], lx[2], lx[3]));
        }
        bf16x8 bh[4], bl[4];
        bfrags(s % kLbBufs, bh, bl);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
          for (int ct = 0; ct < 4; ++ct) {
            acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[rt], bh[ct], acc[rt][ct], 0, 0, 0);
            acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[rt], bl[ct], acc[rt][ct], 0, 0, 0);
            acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[rt], bh[ct], acc[rt][ct], 0, 0, 0);
          }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // the W tiles of step s + 1 (the x loads are waited for already)
        __syncthreads();
      }
    }
    // The last step's barrier: every wavefront is done with the W buffers.
    // Request the next tile's first loads, then store this one.
    const int64_t r0_this = r0;
    const int c0_this = c0;
    const int64_t next = tile + gridDim.x;
    if (next < ntiles) {
      place(next);
      first_loads();
    }
    lb_store_tile<TOut>(acc, stile, a.bias, rs_y, a.m, a.c_out, r0_this + 64 * wr, c0_this + 64 * wc, lane);
  }
}

template <typename TIn>
int launch_lb_d(const LinMfmaArgs& a, const uint32_t* bits, const uint32_t* flags, int cwp, int out_dtype,
                hipStream_t stream) {
  const int64_t tiles = ((a.m + kLbRows - 1) / kLbRows) * ((a.c_out + kLmCols - 1) / kLmCols);
  if (tiles == 0) return (int)hipSuccess;
  // One workgroup per CU (a multiple of 8, at most one per tile rounded up
  // to 8): every CU loops over its tiles.
  const int64_t cus = (num_cus() + 7) / 8 * 8;
  const int64_t grid = tiles < cus ? (tiles + 7) / 8 * 8 : cus;
  if (out_dtype == SF_F32)
    hipLaunchKernelGGL((k_linear_bits_mfma<TIn, float>), dim3((unsigned)grid), dim3(64 * kLbWaves), 0, stream, a,
                       bits, flags, cwp);
  else
    hipLaunchKernelGGL((k_linear_bits_mfma<TIn, TIn>), dim3((unsigned)grid), dim3(64 * kLbWaves), 0, stream, a, bits,
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
