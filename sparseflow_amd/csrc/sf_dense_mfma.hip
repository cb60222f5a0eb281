// Dense-tile branch of the 3x3 pixel-tile Stage 2, on the matrix cores.
//
// The spike walk of k_conv_px3s costs, per 64-pixel wave-tile, as many
// rounds as its busiest pixel has spikes.  Live spiking networks fire in
// bursts: in a direct-encoded Spiking-ResNet50 one time step of sixteen
// carries two thirds of a deep layer's spikes at ~10% density, so a few
// wave-tiles hold most of the work, walk for several times longer than the
// rest and hold their workgroup at every chunk barrier.  Such tiles are dense
// enough for the matrix cores: k_conv_px3s (and the row kernel,
// k_conv_rows_kc, for its row tiles, and the streamed 1x1 walk, k_conv_flat,
// for its pixel tiles) hands them (by a test on the first chunk's words) to a
// per-channel-group queue instead of walking them,
// each as a run of at most 64 output pixels of the flattened (frame, pixel)
// axis, and k_conv_dense_mfma below computes the 64 pixels from each run's
// first (storing the run's own) as an implicit GEMM,
//   y[px, co] = bias[co] + sum_k S[px, k] W[k, co],  k = (tap, ci),
// with the 0/1 spikes exact in bf16 and W split into bf16 hi + lo parts
// (W = hi + lo + O(2^-17 |W|); the 1x1 form adds a third part, exact to
// f32), accumulated in f32: the reference's
// dense-tile tl.dot branch (Kernels/conv2d.py:606-620, the ALL_ONES tile
// class), taken per tile where the tile is dense, not per whole layer.
//
// One workgroup of 8 wavefronts computes four queued tiles of one group at
// a time against 32 of its 64 output channels (a work item: 64 flattened
// output pixels x 32 output channels per tile), its wavefronts specialised:
// four compute wavefronts, one tile each as 4 x 2 MFMA 16x16x32 bf16 tiles
// (the staged B fragments serve all four), and four staging wavefronts,
// which read the weights of the next K chunk (f32, tap-major as every
// Stage-2 kernel takes them, four output channels per load) and the four
// tiles' tap words of that chunk, split the weights into bf16 hi / lo and
// write both to the other half of a double-buffered LDS stage (96 KB, one
// workgroup per CU) while the compute wavefronts run the MFMAs of this one:
// every SIMD holds one wavefront of each kind, the conversion work overlaps
// the matrix cores, the compute wavefronts issue no global loads, and each
// word is loaded once per workgroup, with one barrier per chunk.  Four
// tiles per weight stage stage half the weight bytes per MFMA that two
// tiles of 64 channels would (the weight loads through the CU's vector
// memory path, not the MFMAs, bound this kernel).  The staging runs through
// this workgroup's sequence of (item, chunk) steps without a break between
// items.  A persistent grid takes the items, each XCD those of its own
// 32-channel columns (so a column's weights stay in one L2).  K is walked
// in chunks of 32 input channels x 9 taps; a 32-wide K step is one tap of
// one bitmap word, so a lane's A fragment is 8 bits of a pixel's tap word
// (each lane reads the words of its own fragment rows from the stage)
// turned into bf16 0 / 1 values by a 16-entry nibble table.  Each tap's
// fragments are read while the previous tap's MFMAs run.
//
// Queue state lives in the library's static device memory (one slot per
// stream in use, zero when the code object loads).  The dense kernel runs
// right after k_conv_px3s on the same stream, reads the counts, and its last
// workgroup to finish clears them: every call leaves the slot zero.
#include <map>
#include <mutex>

#include "sf_tile.h"

namespace sf {

static __device__ __align__(256) DenseQueue g_dense_queue[kDenseQueueSlots];

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kDmWaves = 8;                          // wavefronts per workgroup: 4 compute + 4 staging
constexpr int kDmCompute = 4;                        // compute wavefronts (0 .. 3)
constexpr int kDmThreads = 64 * kDmWaves;
constexpr int kDmGroupCo = 64;                       // output channels of a queue group (the pixel-tile kernels' group)
constexpr int kDmCo = 32;                            // output channels of a work item: one column of a group
constexpr int kDmCols = kDmGroupCo / kDmCo;          // work-item columns per group
constexpr int kDmCi = 32;                            // input channels per chunk (one bitmap word)
constexpr int kDmRowsPart = 9 * kDmCo;               // LDS rows (tap, co) of one bf16 part, 64 bytes each
constexpr int kDmStage = kDmRowsPart * kDmCi;        // bf16 elements of one part of one chunk
constexpr int kDmTiles = 4;                          // queued tiles per work item (one per compute wavefront)
constexpr int kDmTapSplit = 5;                       // staging wavefronts 0, 1 take taps 0 .. 4; 2, 3 taps 5 .. 8
constexpr int kDmWLoads = 2 * kDmTapSplit;           // four-channel weight loads per staging thread per chunk (at most)
constexpr int kDmXcds = 8;                           // accelerator complex dies (each with its own L2)

// LDS placement of (row r, 16-byte piece p): row r (64 bytes) sits at line
// dm_row(r) = r ^ (r4 | r2 << 1) (bits of r; the low two bits only, so a
// row stays in its group of four and, rows being tap * 32 + co, the
// placement does not depend on the tap), its piece p at
// p ^ (r2 | (r1 ^ r3) << 1).  Then, for a 128- and a 256-byte bank period
// alike, the rows that one lane group of a fragment read touches (16
// consecutive rows, one piece) fall in distinct 16-byte bank slots, and the
// 4-byte writes of a staging instruction (rows 4 q + j for q = 0 .. 7, two
// neighbouring pieces, four words of each) in distinct banks: neither
// conflicts.
__device__ __forceinline__ int dm_row(int r) { return r ^ (((r >> 4) & 1) | (((r >> 2) & 1) << 1)); }
__device__ __forceinline__ int dm_piece(int r, int p) { return p ^ (((r >> 2) & 1) | ((((r >> 1) ^ (r >> 3)) & 1) << 1)); }

// Two floats to bf16 (round to nearest even) packed in one word, low half =
// v0 (one conversion instruction for the pair).
__device__ __forceinline__ uint32_t dm_bf16x2(float v0, float v1) {
  const bf16x2 h = __builtin_convertvector(f32x2{v0, v1}, bf16x2);
  return __builtin_bit_cast(uint32_t, h);
}

// This workgroup's work items, in order: the items of its XCD's columns
// taken as one sequence (column after column), entries k, k + stride, ...
// of it, so an XCD's workgroups share its columns' items evenly.  Column
// col = 32 output channels (half col % 2) of queue group col / 2; item k of
// a column = its group's queued tiles 4 k .. 4 k + 3.
struct DmItems {
  const int* first;  // LDS: item prefix over the columns
  int cols, cstep, srank, stride;
  int col, k;
  __device__ int nitems(int c) const { return first[c + 1] - first[c]; }
  __device__ void settle() {
    while (col < cols && k >= nitems(col)) {
      k -= nitems(col);
      col += cstep;
    }
  }
  __device__ bool valid() const { return col < cols; }
  __device__ void next() {
    k += stride;
    settle();
  }
};

// ONE: a 1x1 stride-1 convolution (k_conv_flat's dense tiles): the nine K
// steps of a stage are nine consecutive 32-channel words of the pixel's own
// bitmap (pixel-major, as k_conv_flat reads it), and weight row ci (tap-major
// with one tap) holds channel ci; words and rows past C_in read zero through
// the buffer resources' bounds.
template <typename TOut, bool ONE>
__global__ __launch_bounds__(kDmThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_conv_dense_mfma(
    ConvArgs a, DenseQueue* __restrict__ dq, const uint32_t* __restrict__ bits, const float* __restrict__ wt,
    const float* __restrict__ bias_p, TOut* __restrict__ y, int groups, int nchunks) {
  // [stage buffer][part: hi, lo (, lo2)][row (tap, co)][32 ci], pieces
  // swizzled.  The 1x1 form splits W into three bf16 parts (24 bits of
  // mantissa: as exact as the f32 walk, which its tiles replace at every
  // layer of a deep 1x1 stack); the 3x3 form into two.
  constexpr int NPART = ONE ? 3 : 2;
  __shared__ __align__(16) uint16_t s_w[2][NPART][kDmStage];
  // [stage buffer][tile][pixel][tap, padded to 12]: the chunk's bitmap word
  // of each tap of each pixel of the item's tiles (48-byte rows: three
  // aligned 16-byte reads per pixel, sixteen consecutive pixels in distinct
  // banks).
  __shared__ __align__(16) uint32_t s_words[2][kDmTiles][64][12];
  __shared__ __align__(16) uint2 s_tab[16];
  __shared__ int s_first[kDmCols * kDenseQueueGroups + 1];  // items of the columns before column c
  __shared__ int s_tiles[kDenseQueueGroups];                // queued tiles per group
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: roles and scalar row offsets use it
  const int cols = (a.c_out + kDmCo - 1) / kDmCo;  // columns with output channels (at most kDmCols per group)
  // The columns' item counts, read in parallel (one dependent read after
  // another would cost a memory latency each), then their prefix.
  if (tid < cols) {
    const int n = (int)min(dq->count[tid / kDmCols], (uint32_t)kDenseQueueCap);
    if (tid % kDmCols == 0) s_tiles[tid / kDmCols] = n;
    s_first[tid + 1] = (n + kDmTiles - 1) / kDmTiles;
  }
  __syncthreads();
  if (tid == 0) {
    int sum = 0;
    for (int k = 0; k < cols; ++k) {
      const int n = s_first[k + 1];
      s_first[k] = sum;
      sum += n;
    }
    s_first[cols] = sum;
  }
  __syncthreads();
  // Placement: workgroup i runs on XCD i % 8 (the dispatcher's round
  // robin), and each XCD takes the items of one column (columns <= 8: the
  // XCDs of one residue share a column) or of every eighth column, so a
  // column's weights, re-read for every item, stay in one XCD's L2 instead
  // of streaming through all eight.  Correctness does not depend on it.
  const int nrank = (int)gridDim.x / kDmXcds;  // workgroups per XCD (the grid is a multiple of 8)
  const int xcd = (int)blockIdx.x % kDmXcds, rank = (int)blockIdx.x / kDmXcds;
  const int cstep = cols > kDmXcds ? kDmXcds : cols;
  const int share = cols > kDmXcds ? 1 : (kDmXcds - 1 - xcd % cols) / cols + 1;  // XCDs on one column
  const int srank = cols > kDmXcds ? rank : (xcd / cols) * nrank + rank;
  DmItems first_item{s_first, cols, cstep, srank, share * nrank, xcd % cols, srank};
  first_item.settle();
  const bool working = first_item.valid();
  if (working) {
    // Nibble b -> 4 bf16 values, element j = bit j of b ? 1.0 : 0.0 (128
    // bytes: each entry in banks of its own, so a read is conflict-free).
    if (tid < 16) {
      const uint32_t b = (uint32_t)tid;
      s_tab[tid] = make_uint2(((b & 1u) ? 0x3F80u : 0u) | ((b & 2u) ? 0x3F800000u : 0u),
                              ((b & 4u) ? 0x3F80u : 0u) | ((b & 8u) ? 0x3F800000u : 0u));
    }
    if (wave >= kDmCompute) {
      // ---- staging wavefronts ----
      // Thread (q = lane & 7, e = lane >> 3) of staging wavefront v takes
      // output channels 4 q .. 4 q + 3 of the column (one 16-byte load; 8
      // lanes read a 128-byte run of a weight row) and input channels 2 p,
      // 2 p + 1 of the chunk, p = e + 8 (v & 1), taps 0 .. 4 (v < 2) or
      // 5 .. 8: 4 bytes (one bf16 pair) of piece p / 4 of each of its rows.
      // The wave-uniform part of the row offset rides in the load's scalar
      // offset.  At most 10 loads per chunk, plus the 9 tap words of pixel
      // t*64 + lane of tile v of the item: two chunks' loads fit in the
      // memory counter (63).
      const int sv = wave - kDmCompute;
      const int cq = lane & 7, ce = lane >> 3;
      const int cpair = ce + 8 * (sv & 1);             // input-channel pair of the chunk
      const int tap0 = (sv >> 1) * kDmTapSplit;        // wave-uniform
      const int ntap = sv >> 1 ? 9 - kDmTapSplit : kDmTapSplit;
      const int row4 = a.c_out * 4;
      const auto rs_w = buf_rsrc(wt, (uint32_t)((int64_t)a.c_in * (ONE ? 1 : 9) * a.c_out * 4));
      // Lanes past the last queued tile take the item's first tile (their
      // rows are computed and never stored).
      const int hwo = a.hw_out;
      const int total_px = (int)(a.n * hwo);
      const uint32_t frame_bytes = (uint32_t)a.hw_in * (uint32_t)a.cwp * 4u;
      const auto rs_bits = buf_rsrc(bits, (uint32_t)((int64_t)a.n * frame_bytes));
      int ih0 = 0, iw0 = 0, qpx = 0;
      uint32_t fbase = 0;
      auto item_pixel = [&](const DmItems& p) {
        const int grp = p.col / kDmCols;
        const int e0 = kDmTiles * p.k;
        const int e = e0 + sv < s_tiles[grp] ? e0 + sv : e0;
        const int gp = (int)dq->start[grp][e] + lane;
        const int gc = gp < total_px ? gp : total_px - 1;
        const int sample = gc / hwo;
        const int q = gc - sample * hwo;
        const int oh = q / a.w_out, ow = q - oh * a.w_out;
        ih0 = oh * a.s - 1;
        iw0 = ow * a.s - 1;
        qpx = q;
        fbase = (uint32_t)sample * frame_bytes;
      };
      auto load_w = [&](f32x4 (&wv)[kDmWLoads], int col, int c) {
        const int co0 = (col / kDmCols) * kDmGroupCo + (col % kDmCols) * kDmCo;
        const int wcol = co0 + 4 * cq < a.c_out ? co0 + 4 * cq : a.c_out - 4;  // c_out is a multiple of 4
        if constexpr (ONE) {
          // Step tp of stage c: word w = 9 c + tap0 + tp, channels 32 w + 16 (v & 1)
          // + 2 e + j (rows past C_in read zero).
          uint32_t vo = (uint32_t)wcol * 4u + (uint32_t)(2 * ce * row4);
          asm volatile("" : "+v"(vo));
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            int so = ((9 * c + tap0) * 32 + 16 * (sv & 1) + j) * row4;
#pragma unroll
            for (int tp = 0; tp < kDmTapSplit; ++tp) {
              if (tp < ntap) {
                asm volatile("" : "+s"(so));
                wv[j * kDmTapSplit + tp] =
                    __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_w, (int)vo, so, 0));
                so += 32 * row4;
              }
            }
          }
          return;
        }
        uint32_t vo = (uint32_t)wcol * 4u + (uint32_t)(2 * ce * 9 * row4);
        asm volatile("" : "+v"(vo));
        // One scalar offset register stepped by a row (opaque, so the row
        // offsets are not precomputed into scalar registers, which spills).
        const int ci0 = c * kDmCi + 16 * (sv & 1);  // wave-uniform; this lane's channels are ci0 + 2 e + {0, 1}
        if (ci0 + 16 <= a.c_in) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            int so = ((ci0 + j) * 9 + tap0) * row4;
#pragma unroll
            for (int tp = 0; tp < kDmTapSplit; ++tp) {
              if (tp < ntap) {
                asm volatile("" : "+s"(so));
                wv[j * kDmTapSplit + tp] =
                    __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_w, (int)vo, so, 0));
                so += row4;
              }
            }
          }
        } else {
          // The last, partial chunk: channels past C_in are zero rows.
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const bool live = ci0 + 2 * ce + j < a.c_in;
            int so = ((ci0 + j) * 9 + tap0) * row4;
#pragma unroll
            for (int tp = 0; tp < kDmTapSplit; ++tp) {
              if (tp < ntap) {
                asm volatile("" : "+s"(so));
                wv[j * kDmTapSplit + tp] =
                    live ? __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_w, (int)vo, so, 0))
                         : f32x4{0.f, 0.f, 0.f, 0.f};
                so += row4;
              }
            }
          }
        }
      };
      // Row r = tap * 32 + 4 q + j of a part: its 4 bytes for this thread
      // sit at a per-lane base plus a constant (bits 0 .. 4 of r come from
      // 4 q + j alone).
      auto store_w = [&](int sb, const f32x4 (&wv)[kDmWLoads], const uint32_t (&wd)[9]) {
        uint32_t* row = s_words[sb][sv][lane];
        *reinterpret_cast<uint4*>(row) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
        *reinterpret_cast<uint4*>(row + 4) = make_uint4(wd[4], wd[5], wd[6], wd[7]);
        row[8] = wd[8];
        uint16_t* sh = s_w[sb][0];
        uint16_t* sl = s_w[sb][1];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r0 = 4 * cq + j;
          const int el0 = dm_row(r0) * kDmCi + 8 * dm_piece(r0, cpair >> 2) + 2 * (cpair & 3);
#pragma unroll
          for (int tp = 0; tp < kDmTapSplit; ++tp) {
            if (tp < ntap) {
              const float v0 = wv[tp][j], v1 = wv[kDmTapSplit + tp][j];
              const uint32_t hi = dm_bf16x2(v0, v1);
              // Residues exact in f32 (each part is its value rounded).
              const float r0 = v0 - __uint_as_float(hi << 16), r1 = v1 - __uint_as_float(hi & 0xFFFF0000u);
              const uint32_t lo = dm_bf16x2(r0, r1);
              const int el = el0 + (tap0 + tp) * kDmCo * kDmCi;
              *reinterpret_cast<uint32_t*>(&sh[el]) = hi;
              *reinterpret_cast<uint32_t*>(&sl[el]) = lo;
              if constexpr (ONE) {
                const uint32_t lo2 =
                    dm_bf16x2(r0 - __uint_as_float(lo << 16), r1 - __uint_as_float(lo & 0xFFFF0000u));
                *reinterpret_cast<uint32_t*>(&s_w[sb][NPART - 1][el]) = lo2;
              }
            }
          }
        }
      };
      // Steps (item, chunk) in the compute wavefronts' order; `ld` is the
      // next step to load.  Two register sets: a step's loads are issued a
      // whole step before they are converted and written (the wait for them
      // overlaps the other set's conversion and the compute wavefronts'
      // MFMAs).
      DmItems ld = first_item;
      int ldc = 0;
      auto load = [&](f32x4 (&wv)[kDmWLoads], uint32_t (&wd)[9]) {
        if constexpr (ONE) {
#pragma unroll
          for (int t = 0; t < 9; ++t) {
            const int w = 9 * ldc + t;
            const uint32_t off = w < a.cwp ? fbase + (uint32_t)(qpx * a.cwp + w) * 4u : 0x80000000u;
            wd[t] = __builtin_amdgcn_raw_buffer_load_b32(rs_bits, (int)off, 0, 0);
          }
        } else {
          px3_load_words_at(wd, rs_bits, fbase, a, ih0, iw0, ldc);
        }
        load_w(wv, ld.col, ldc);
        if (++ldc == nchunks) {
          ldc = 0;
          ld.next();
          if (ld.valid()) item_pixel(ld);
        }
      };
      f32x4 wa[kDmWLoads], wb[kDmWLoads];
      uint32_t da[9], db[9];
      item_pixel(ld);
      load(wa, da);  // step 0
      bool h1 = ld.valid();
      if (h1) load(wb, db);  // step 1
      store_w(0, wa, da);
      __syncthreads();  // stage 0 (and the table) written
      // One barrier per step, as the compute wavefronts: during step st
      // (computed from stage st & 1) load step st + 2 and stage step st + 1.
      for (int st = 0;; st += 2) {
        bool h2 = false;
        if (h1) {
          h2 = ld.valid();
          if (h2) load(wa, da);
          store_w((st + 1) & 1, wb, db);
        }
        __syncthreads();
        if (!h1) break;
        bool h3 = false;
        if (h2) {
          h3 = ld.valid();
          if (h3) load(wb, db);
          store_w(st & 1, wa, da);  // stage (st + 2) & 1
        }
        __syncthreads();
        if (!h2) break;
        h1 = h3;
      }
    } else {
      // ---- compute wavefronts ----
      // Compute wavefront w takes tile w of each item: 64 pixels x the
      // column's 32 output channels, as 4 x 2 MFMA 16x16x32 bf16 tiles (the
      // four wavefronts read the same B fragments).
      const int hwo = a.hw_out;
      const int total_px = (int)(a.n * hwo);
      const int li = lane & 15, g = lane >> 4;
      __syncthreads();  // stage 0 written
      int st = 0;
      for (DmItems it = first_item; it.valid(); it.next()) {
        const int grp = it.col / kDmCols;
        const int e0 = kDmTiles * it.k;
        const bool has = e0 + wave < s_tiles[grp];
        const int p0 = (int)dq->start[grp][has ? e0 + wave : e0];  // the run's first output pixel
        const int npx = has ? (int)dq->npx[grp][e0 + wave] : 0;
        const int co0 = grp * kDmGroupCo + (it.col % kDmCols) * kDmCo;
        f32x4 acc[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int c = 0; c < nchunks; ++c, ++st) {
          // The tap words of this lane's fragment rows: pixel 16 rt + li of
          // the tile.
          uint32_t w[4][9];
#pragma unroll
          for (int rt = 0; rt < 4; ++rt) {
            const uint32_t* row = s_words[st & 1][wave][16 * rt + li];
            const uint4 q0 = *reinterpret_cast<const uint4*>(row);
            const uint4 q1 = *reinterpret_cast<const uint4*>(row + 4);
            const uint4 q2 = *reinterpret_cast<const uint4*>(row + 8);
            w[rt][0] = q0.x, w[rt][1] = q0.y, w[rt][2] = q0.z, w[rt][3] = q0.w;
            w[rt][4] = q1.x, w[rt][5] = q1.y, w[rt][6] = q1.z, w[rt][7] = q1.w;
            w[rt][8] = q2.x;
          }
          const uint16_t* sh = s_w[st & 1][0];
          const uint16_t* sl = s_w[st & 1][1];
          const uint16_t* sl2 = s_w[st & 1][NPART - 1];
          bf16x8 bh[2][2], bl[2][2], bl2[2][2], af[2][4];
          auto frags = [&](int tap, int bb) {
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
              const int r = tap * kDmCo + 16 * ct + li;
              const int off = dm_row(r) * kDmCi + 8 * dm_piece(r, g);
              bh[bb][ct] = *reinterpret_cast<const bf16x8*>(&sh[off]);
              bl[bb][ct] = *reinterpret_cast<const bf16x8*>(&sl[off]);
              if constexpr (ONE) bl2[bb][ct] = *reinterpret_cast<const bf16x8*>(&sl2[off]);
            }
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
              // Row 16 rt + li of the tile: that pixel's tap word, bits 8g .. 8g+7.
              const uint32_t byte = __builtin_amdgcn_ubfe(w[rt][tap], 8 * g, 8);
              const uint2 lo = s_tab[byte & 15u], hi = s_tab[byte >> 4];
              af[bb][rt] = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
            }
          };
          frags(0, 0);
#pragma unroll
          for (int tap = 0; tap < 9; ++tap) {
            __builtin_amdgcn_sched_barrier(0);
            const int cb = tap & 1;
            if (tap + 1 < 9) frags(tap + 1, cb ^ 1);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt)
#pragma unroll
              for (int ct = 0; ct < 2; ++ct)
                acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[cb][rt], bh[cb][ct], acc[rt][ct], 0, 0, 0);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt)
#pragma unroll
              for (int ct = 0; ct < 2; ++ct)
                acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[cb][rt], bl[cb][ct], acc[rt][ct], 0, 0, 0);
            if constexpr (ONE) {
#pragma unroll
              for (int rt = 0; rt < 4; ++rt)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
                  acc[rt][ct] =
                      __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[cb][rt], bl2[cb][ct], acc[rt][ct], 0, 0, 0);
            }
          }
          __syncthreads();  // stage st & 1 free for step st + 2; stage (st + 1) & 1 written
        }
        // Accumulator (rt, ct) element i of lane (li, g): output pixel
        // p0 + 16 rt + 4 g + i (stored for the run's first npx), output
        // channel co0 + 16 ct + li.
        if (has) {
          float bv[2];
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) {
            const int co = co0 + 16 * ct + li;
            bv[ct] = bias_p != nullptr && co < a.c_out ? bias_p[co] : 0.f;
          }
#pragma unroll
          for (int rt = 0; rt < 4; ++rt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int pix = p0 + 16 * rt + 4 * g + i;
              if (16 * rt + 4 * g + i >= npx || pix >= total_px) continue;
              const int smp = pix / hwo;
              const int64_t ybase = (int64_t)smp * a.c_out * hwo + (pix - smp * hwo);
#pragma unroll
              for (int ct = 0; ct < 2; ++ct) {
                const int co = co0 + 16 * ct + li;
                if (co >= a.c_out) continue;
                y[ybase + (int64_t)co * hwo] = from_f32<TOut>(acc[rt][ct][i] + bv[ct]);
              }
            }
        }
      }
    }
  }
  // The last workgroup with items to finish clears the slot for the next
  // call: every such workgroup read the counts (and waited for them) before
  // its own atomic, and the atomics on `done` are ordered, so the clearing
  // follows each of their reads.  A workgroup without items may read the
  // counts before or after the clearing: either way it has nothing to do,
  // and it takes no part (with an empty queue nothing is counted or
  // cleared).  No fence: the next kernel on the stream sees the stores.
  if (working) {
    // Workgroups with items, the same count in every workgroup: per XCD, the
    // ranks below its columns' item count (less the ranks of the XCDs before
    // it on the same column).
    int nworking = 0;
    for (int x = 0; x < kDmXcds; ++x) {
      int items = 0;
      for (int col = x % cols; col < cols; col += cstep) items += s_first[col + 1] - s_first[col];
      const int before = cols > kDmXcds ? 0 : (x / cols) * nrank;
      nworking += min(max(items - before, 0), nrank);
    }
    __syncthreads();
    if (tid == 0 && atomicAdd(&dq->done, 1u) == (uint32_t)nworking - 1) {
      for (int k = 0; k < groups; ++k) dq->count[k] = 0u;
      dq->done = 0u;
    }
  }
}

// Per-device table of stream -> queue slot (the first kDenseQueueSlots
// streams that launch a deferring kernel on a device each get a slot).
constexpr int kDqMaxDevices = 64;
std::mutex g_dq_mu;
DenseQueue* g_dq_base[kDqMaxDevices] = {};
std::map<uintptr_t, int> g_dq_slot[kDqMaxDevices];

}  // namespace

namespace {

// The queue array's device address on GPU `dev` (looked up once per GPU,
// with it current); nullptr if the lookup fails.  Caller holds g_dq_mu.
DenseQueue* dq_base_locked(int dev) {
  if (g_dq_base[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_dense_queue)) != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      return nullptr;
    }
    g_dq_base[dev] = static_cast<DenseQueue*>(p);
  }
  return g_dq_base[dev];
}

}  // namespace

int dense_queue_prepare() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kDqMaxDevices) return (int)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_dq_mu);
  return dq_base_locked(dev) != nullptr ? (int)hipSuccess : (int)hipErrorInvalidSymbol;
}

DenseQueue* dense_queue_for(hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDqMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lk(g_dq_mu);
  if (dq_base_locked(dev) == nullptr) return nullptr;
  auto& slots = g_dq_slot[dev];
  const uintptr_t key = reinterpret_cast<uintptr_t>(stream);
  auto it = slots.find(key);
  if (it == slots.end()) {
    if ((int)slots.size() >= kDenseQueueSlots) return nullptr;  // no deferral on this stream
    it = slots.emplace(key, (int)slots.size()).first;
  }
  return g_dq_base[dev] + it->second;
}

int launch_conv_dense_mfma(const ConvArgs& a, DenseQueue* dq, int out_dtype, hipStream_t stream) {
  const int groups = (a.c_out + kDmGroupCo - 1) / kDmGroupCo;
  if (groups > kDenseQueueGroups) return (int)hipErrorInvalidValue;
  const bool one = a.k == 1;
  // Stages: 32-channel chunks (3x3, nine taps each), or groups of nine
  // 32-channel words (1x1).
  const int nchunks = one ? (a.cwp + 8) / 9 : (a.c_in + kDmCi - 1) / kDmCi;
  // One workgroup per CU (the stage fills most of its LDS; the queue sizes
  // are known only on the device, and workgroups without items read the
  // counts and leave).
  const int grid = (num_cus() + kDmXcds - 1) / kDmXcds * kDmXcds;
  timing_begin(K_DENSE_MFMA, stream);
  auto go = [&](auto kern, auto* yp) {
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kDmThreads), 0, stream, a, dq, a.bits, a.wt, a.bias, yp, groups, nchunks);
  };
  if (out_dtype == SF_F16) {
    if (one) go(k_conv_dense_mfma<__half, true>, static_cast<__half*>(a.y));
    else go(k_conv_dense_mfma<__half, false>, static_cast<__half*>(a.y));
  } else if (out_dtype == SF_BF16) {
    if (one) go(k_conv_dense_mfma<__hip_bfloat16, true>, static_cast<__hip_bfloat16*>(a.y));
    else go(k_conv_dense_mfma<__hip_bfloat16, false>, static_cast<__hip_bfloat16*>(a.y));
  } else {
    if (one) go(k_conv_dense_mfma<float, true>, static_cast<float*>(a.y));
    else go(k_conv_dense_mfma<float, false>, static_cast<float*>(a.y));
  }
  const int rc = (int)hipGetLastError();
  timing_end(K_DENSE_MFMA, stream);
  return rc;
}

}  // namespace sf
