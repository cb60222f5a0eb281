// C ABI of libsparseflow_hip.so: argument validation, workspace layout,
// launch sequencing and per-kernel event timing.  See include/sparseflow.h.
#include <math.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "sf_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(int rc, const char* what) {
  return fail(SF_ERR_HIP, std::string(what) + ": " + hipGetErrorString((hipError_t)rc));
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// ---- IEEE binary16 round-to-nearest-even, host side ------------------------

uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));  // inf / NaN
  const int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);  // overflow -> inf
  if (e <= 0) {
    // Subnormal (or zero) half: value = man_full * 2^(exp-150); unit 2^-24.
    if (e < -10) return (uint16_t)sign;  // below half of the smallest subnormal
    man |= 0x800000u;
    const int shift = 14 - e;  // bits to drop so the unit becomes 2^-24
    uint32_t q = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // carries into the exponent correctly
  return (uint16_t)h;
}

float f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  float out;
  if (exp == 0) {
    out = ldexpf((float)man, -24);
    if (sign) out = -out;
    return out;
  }
  if (exp == 31) {
    uint32_t x = sign | 0x7f800000u | (man << 13);
    memcpy(&out, &x, 4);
    return out;
  }
  uint32_t x = sign | ((exp - 15 + 127) << 23) | (man << 13);
  memcpy(&out, &x, 4);
  return out;
}

float f16_round(float f) { return f16_bits_to_f32(f32_to_f16_bits(f)); }

// ---- validation ------------------------------------------------------------

bool dtype_ok(int d) { return d == SF_F32 || d == SF_F16 || d == SF_BF16; }

int check_desc(const sf_conv_desc* d, bool allow_k1s2 = true) {
  if (d == nullptr) return fail(SF_ERR_INVALID, "desc is NULL");
  if (d->n < 0) return fail(SF_ERR_INVALID, "n < 0");
  if (d->c_in < 1 || d->h_in < 1 || d->w_in < 1 || d->c_out < 1 || d->h_out < 1 || d->w_out < 1)
    return fail(SF_ERR_INVALID, "non-positive dimension");
  if (!dtype_ok(d->in_dtype) || !dtype_ok(d->out_dtype)) return fail(SF_ERR_INVALID, "unknown dtype");
  if (d->out_dtype != d->in_dtype && d->out_dtype != SF_F32)
    return fail(SF_ERR_UNSUPPORTED, "out_dtype must equal in_dtype or be f32");
  const bool k3 = d->kernel == 3 && d->pad == 1 && (d->stride == 1 || d->stride == 2);
  const bool k1 = d->kernel == 1 && d->pad == 0 && (d->stride == 1 || (allow_k1s2 && d->stride == 2));
  if (!k3 && !k1) return fail(SF_ERR_UNSUPPORTED, "supported patterns: 3x3 s1/s2 p1, 1x1 s1 p0");
  const int ho = (d->h_in + 2 * d->pad - d->kernel) / d->stride + 1;
  const int wo = (d->w_in + 2 * d->pad - d->kernel) / d->stride + 1;
  if (ho != d->h_out || wo != d->w_out) return fail(SF_ERR_INVALID, "h_out/w_out do not match the conv geometry");
  if (sf::words_per_pixel(d->c_in) > 64) return fail(SF_ERR_UNSUPPORTED, "c_in > 2048");
  if ((int64_t)d->h_in * d->w_in > (1 << 30))
    return fail(SF_ERR_UNSUPPORTED, "tensor too large for 32-bit in-frame offsets");
  // Stage-2 list entries pack a weight-row byte offset into 26 bits.
  if ((int64_t)d->c_in * d->kernel * d->kernel * d->c_out * 4 > (1ll << 26))
    return fail(SF_ERR_UNSUPPORTED, "weights larger than 64 MiB");
  // The per-wavefront entry list must hold a pixel's worst case in LDS.
  sf::ConvArgs g{};
  g.c_in = d->c_in;
  g.h_in = d->h_in;
  g.w_in = d->w_in;
  g.c_out = d->c_out;
  g.h_out = d->h_out;
  g.w_out = d->w_out;
  g.k = d->kernel;
  g.cwp = sf::words_per_pixel(d->c_in);
  sf::conv_geometry(g, true);
  const int lif_lds = g.wave_lds;
  sf::conv_geometry(g, false);
  if (g.wave_lds > sf::kMaxLdsBytes || lif_lds > sf::kMaxLdsBytes)
    return fail(SF_ERR_UNSUPPORTED, "c_in too wide for this kernel (per-wavefront LDS list exceeds 160 KB)");
  return SF_OK;
}

struct Workspace {
  uint32_t* bits;
  uint32_t* flags;
  size_t bytes;
};

Workspace carve(void* ws, int64_t frames, int c, int h, int w) {
  Workspace out{};
  const size_t bits_b = align256(sf_prescan_bitmap_bytes(frames, c, h, w));
  const size_t flags_b = align256(sf_prescan_flags_bytes(frames, c, h, w));
  out.bits = static_cast<uint32_t*>(ws);
  out.flags = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + bits_b);
  out.bytes = bits_b + flags_b;
  return out;
}

sf::PackArgs pack_args(const void* x, int64_t n, int c, int h, int w, float threshold, uint32_t* bits,
                       uint32_t* flags) {
  const sf::PackPlan pl = sf::make_pack_plan(n, c, h, w);
  sf::PackArgs a{};
  a.x = x;
  a.bits = bits;
  a.flags = flags;
  a.n = n;
  a.c = c;
  a.hw = h * w;
  a.cwp = pl.cwp;
  a.csplit = pl.csplit;
  a.vec = pl.vec;
  a.chunks_per_frame = pl.chunks_per_frame;
  a.total_chunks = pl.total_chunks;
  a.cutoff = sf_activity_cutoff(threshold);
  return a;
}

sf::ConvArgs conv_args(const sf_conv_desc* d, int64_t frames, const uint32_t* bits, const uint32_t* flags,
                       const void* x, const float* wt, const float* bias, void* y, bool lif) {
  const sf::PackPlan pl = sf::make_pack_plan(frames, d->c_in, d->h_in, d->w_in);
  sf::ConvArgs a{};
  a.bits = bits;
  a.flags = flags;
  a.x = x;
  a.wt = wt;
  a.bias = bias;
  a.y = y;
  a.n = d->n;
  a.c_in = d->c_in;
  a.h_in = d->h_in;
  a.w_in = d->w_in;
  a.c_out = d->c_out;
  a.h_out = d->h_out;
  a.w_out = d->w_out;
  a.k = d->kernel;
  a.s = d->stride;
  a.p = d->pad;
  a.cwp = pl.cwp;
  a.bm_ps = pl.cwp;  // the [hw][cwp] words of sf_prescan_pack
  a.bm_ws = 1;
  a.chunk = pl.chunk;
  a.chunks_per_frame = pl.chunks_per_frame;
  a.T = 1;
  sf::conv_geometry(a, lif);
  a.total_groups = d->n * (int64_t)a.groups_per_frame;
  return a;
}

// ---- Stage 2 selection ----------------------------------------------------------

enum class Stage2 { kMfma, kBand, kRowsKc, kPx3, kFlat, kGather };

Stage2 pick_stage2(const sf_conv_desc* d, const sf::ConvArgs& a) {
  // 3x3 with a reduction of at most 32 (an image stem): one dense tile on the
  // matrix cores, whatever the density.
  if (d->in_dtype == SF_F32 && sf::mfma_conv_applicable(a)) return Stage2::kMfma;
  if (sf::band_applicable(a)) return Stage2::kBand;
  // The row-band kernel where the pixel-tile kernel would have to stream its
  // weights (C_in > 128 at 28x28 / 14x14); measured faster there, slower
  // where the pixel-tile weights stay resident.
  if (sf::rows_kc_applicable(a) && !(sf::px3_applicable(a) && sf::px3_resident(a))) return Stage2::kRowsKc;
  if (sf::px3_applicable(a)) return Stage2::kPx3;
  if (sf::flat_applicable(a)) return Stage2::kFlat;
  return Stage2::kGather;
}

int run_stage2(Stage2 k, const sf_conv_desc* d, const sf::ConvArgs& a, void* stream) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  int rc = hipSuccess;
  const char* what = "conv_gather launch";
  switch (k) {
    case Stage2::kMfma: rc = sf::launch_conv_mfma(a, d->in_dtype, d->out_dtype, st); what = "conv_mfma launch"; break;
    case Stage2::kBand: rc = sf::launch_conv_band(a, d->in_dtype, d->out_dtype, st); what = "conv_rows launch"; break;
    case Stage2::kRowsKc:
      rc = sf::launch_conv_rows_kc(a, d->in_dtype, d->out_dtype, st);
      what = "conv_rows_kc launch";
      break;
    case Stage2::kPx3: rc = sf::launch_conv_px3(a, d->in_dtype, d->out_dtype, st); what = "conv_px3 launch"; break;
    case Stage2::kFlat: rc = sf::launch_conv_flat(a, d->in_dtype, d->out_dtype, st); what = "conv_flat launch"; break;
    case Stage2::kGather: rc = sf::launch_conv(a, d->in_dtype, d->out_dtype, st); break;
  }
  if (rc != hipSuccess) return hip_fail(rc, what);
  return SF_OK;
}

// Whether the Stage 2 kernel reads word planes ([frame][cwp][hw]): the
// pixel-tile and K-chunked row kernels load one bitmap word of 64
// neighbouring pixels at a time; every other Stage 2 kernel reads the
// [hw][cwp] words of sf_prescan_pack.
bool reads_planes(Stage2 k) { return k == Stage2::kPx3 || k == Stage2::kRowsKc; }

// Prescan into word planes or pixel-major words.
int prescan_for(const sf_conv_desc* d, int64_t frames, const void* x, float threshold, bool planar, uint32_t* bits,
                uint32_t* flags, void* stream) {
  sf::PackArgs pa = pack_args(x, frames, d->c_in, d->h_in, d->w_in, threshold, bits, flags);
  pa.planar = planar ? 1 : 0;
  const int rc = sf::launch_pack(pa, d->in_dtype, static_cast<hipStream_t>(stream));
  if (rc != hipSuccess) return hip_fail(rc, "prescan_pack launch");
  return SF_OK;
}

void use_planes(sf::ConvArgs& a) {
  a.bm_ps = 1;
  a.bm_ws = a.hw_in;
}

// ---- timing -----------------------------------------------------------------

struct TimingRec {
  int id;
  hipEvent_t start, end;
};

std::mutex g_tmu;
bool g_timing = false;
std::vector<TimingRec> g_pending;
double g_total_ms[sf::K_COUNT] = {};
int64_t g_count[sf::K_COUNT] = {};
const char* g_names[sf::K_COUNT] = {"prescan_pack", "prescan_tiles", "conv_gather", "conv_lif", "conv_rows",
                                     "conv_rows_kc", "conv_flat", "conv_px3", "conv_lif_px3",
                                     "lif_multistep", "prescan_rows", "linear_flat", "bmm_sparse",
                                     "spike_attention", "linear_mfma", "bmm_mfma", "conv_lif_flat", "conv_mfma",
                                     "conv_rows_fused", "conv_dense_mfma"};

}  // namespace

namespace sf {

void timing_begin(int kernel_id, hipStream_t stream) {
  std::lock_guard<std::mutex> lk(g_tmu);
  if (!g_timing) return;
  TimingRec r{kernel_id, nullptr, nullptr};
  if (hipEventCreate(&r.start) != hipSuccess) return;
  (void)hipEventRecord(r.start, stream);
  g_pending.push_back(r);
}

void timing_end(int kernel_id, hipStream_t stream) {
  std::lock_guard<std::mutex> lk(g_tmu);
  if (!g_timing) return;
  for (auto it = g_pending.rbegin(); it != g_pending.rend(); ++it) {
    if (it->id == kernel_id && it->end == nullptr) {
      if (hipEventCreate(&it->end) == hipSuccess) (void)hipEventRecord(it->end, stream);
      return;
    }
  }
}

}  // namespace sf

extern "C" {

int sf_version(void) { return 101; }

const char* sf_last_error(void) { return g_last_error.c_str(); }

float sf_activity_cutoff(float threshold) {
  if (isnan(threshold)) return NAN;
  const float th = f16_round(threshold);
  if (isinf(th) && th > 0) return NAN;  // no half exceeds +inf: nothing is active
  if (th < 0.f) return 0.f;              // every non-NaN |v| rounds to >= 0 > th
  // Smallest non-negative float f with f16(f) > th; f16 rounding is monotone,
  // so bisect over the ordered bit patterns of non-negative floats.
  uint32_t lo = 0u, hi = 0x7f800000u;  // f16(+inf) = inf > th
  while (lo < hi) {
    const uint32_t mid = lo + (hi - lo) / 2;
    float f;
    memcpy(&f, &mid, 4);
    if (f16_round(f) > th) hi = mid; else lo = mid + 1;
  }
  float out;
  memcpy(&out, &lo, 4);
  return out;
}

int sf_bitmap_words_per_pixel(int32_t c) { return c < 1 ? 0 : sf::words_per_pixel(c); }

int32_t sf_prescan_chunk_pixels(int64_t n, int32_t c, int32_t h, int32_t w) {
  if (n <= 0 || c < 1 || h < 1 || w < 1) return 0;
  return sf::make_pack_plan(n, c, h, w).chunk;
}

size_t sf_prescan_bitmap_bytes(int64_t n, int32_t c, int32_t h, int32_t w) {
  if (n <= 0 || c < 1 || h < 1 || w < 1) return 0;
  return (size_t)n * (size_t)h * (size_t)w * (size_t)sf::words_per_pixel(c) * 4u;
}

size_t sf_prescan_flags_bytes(int64_t n, int32_t c, int32_t h, int32_t w) {
  if (n <= 0 || c < 1 || h < 1 || w < 1) return 0;
  return (size_t)sf::make_pack_plan(n, c, h, w).total_chunks * 4u;
}

size_t sf_conv2d_workspace_size(const sf_conv_desc* d) {
  if (d == nullptr || d->n <= 0) return 0;
  return align256(sf_prescan_bitmap_bytes(d->n, d->c_in, d->h_in, d->w_in)) +
         align256(sf_prescan_flags_bytes(d->n, d->c_in, d->h_in, d->w_in));
}

size_t sf_conv_lif_workspace_size(const sf_conv_desc* d, int32_t T) {
  if (d == nullptr || d->n <= 0 || T <= 0) return 0;
  const int64_t frames = d->n * (int64_t)T;
  return align256(sf_prescan_bitmap_bytes(frames, d->c_in, d->h_in, d->w_in)) +
         align256(sf_prescan_flags_bytes(frames, d->c_in, d->h_in, d->w_in));
}

int sf_prescan_pack(const void* x, int32_t dtype, int64_t n, int32_t c, int32_t h, int32_t w, float threshold,
                    uint32_t* bits, uint32_t* flags, void* stream) {
  if (n < 0 || c < 1 || h < 1 || w < 1) return fail(SF_ERR_INVALID, "bad prescan shape");
  if (!dtype_ok(dtype)) return fail(SF_ERR_INVALID, "unknown dtype");
  if (sf::words_per_pixel(c) > 64) return fail(SF_ERR_UNSUPPORTED, "c > 2048");
  if ((int64_t)h * w > (1 << 30)) return fail(SF_ERR_UNSUPPORTED, "plane too large");
  if (n == 0) return SF_OK;
  if (x == nullptr || bits == nullptr || flags == nullptr) return fail(SF_ERR_INVALID, "NULL pointer");
  const sf::PackArgs a = pack_args(x, n, c, h, w, threshold, bits, flags);
  const int rc = sf::launch_pack(a, dtype, static_cast<hipStream_t>(stream));
  if (rc != hipSuccess) return hip_fail(rc, "prescan_pack launch");
  return SF_OK;
}

int sf_prescan_tiles(const uint32_t* bits, int64_t n, int32_t c, int32_t h_in, int32_t w_in, int32_t h_out,
                     int32_t w_out, int32_t kernel, int32_t stride, int32_t pad, int32_t tile_h, int32_t tile_w,
                     int32_t group_size, uint32_t* ch_mask, int32_t* ch_count, int32_t* ch_list, int32_t* ag_mask,
                     int32_t* tile_class, void* stream) {
  if (n < 0 || c < 1 || h_in < 1 || w_in < 1 || h_out < 1 || w_out < 1 || tile_h < 1 || tile_w < 1)
    return fail(SF_ERR_INVALID, "bad tiles shape");
  if (kernel < 1 || stride < 1 || pad < 0 || kernel < stride)
    return fail(SF_ERR_UNSUPPORTED, "receptive field must be contiguous (kernel >= stride)");
  if ((h_in + 2 * pad - kernel) / stride + 1 != h_out || (w_in + 2 * pad - kernel) / stride + 1 != w_out)
    return fail(SF_ERR_INVALID, "h_out/w_out do not match the geometry");
  const int cwp = sf::words_per_pixel(c);
  if (cwp > 64) return fail(SF_ERR_UNSUPPORTED, "c > 2048");
  const bool want_groups = ag_mask != nullptr || tile_class != nullptr;
  int ngroups = 0;
  if (want_groups) {
    if (group_size < 16 || (group_size & (group_size - 1)) != 0)
      return fail(SF_ERR_UNSUPPORTED, "group_size must be a power of two >= 16");
    ngroups = (c + group_size - 1) / group_size;
    if (ngroups > 32) return fail(SF_ERR_UNSUPPORTED, "more than 32 channel groups");
  }
  if (n == 0) return SF_OK;
  if (bits == nullptr) return fail(SF_ERR_INVALID, "bits is NULL");
  sf::TilesArgs a{};
  a.bits = bits;
  a.ch_mask = ch_mask;
  a.ch_count = ch_count;
  a.ch_list = ch_list;
  a.ag_mask = ag_mask;
  a.tile_class = tile_class;
  a.n = n;
  a.c = c;
  a.cwp = cwp;
  a.h_in = h_in;
  a.w_in = w_in;
  a.h_out = h_out;
  a.w_out = w_out;
  a.k = kernel;
  a.s = stride;
  a.p = pad;
  a.th = tile_h;
  a.tw = tile_w;
  a.gh = (h_out + tile_h - 1) / tile_h;
  a.gw = (w_out + tile_w - 1) / tile_w;
  a.group_size = group_size;
  a.ngroups = ngroups;
  a.ntiles = n * (int64_t)a.gh * a.gw;
  const int rc = sf::launch_tiles(a, static_cast<hipStream_t>(stream));
  if (rc != hipSuccess) return hip_fail(rc, "prescan_tiles launch");
  return SF_OK;
}

int sf_conv2d_sparse(const sf_conv_desc* d, const uint32_t* bits, const uint32_t* flags, const void* x,
                     const float* wt, const float* bias, void* y, void* stream) {
  int rc = check_desc(d);
  if (rc != SF_OK) return rc;
  if (d->n == 0) return SF_OK;
  if (bits == nullptr || flags == nullptr || x == nullptr || wt == nullptr || y == nullptr)
    return fail(SF_ERR_INVALID, "NULL pointer");
  const sf::ConvArgs a = conv_args(d, d->n, bits, flags, x, wt, bias, y, false);
  return run_stage2(pick_stage2(d, a), d, a, stream);
}

int sf_conv2d_bitmap_layout(const sf_conv_desc* d) {
  const int rc = check_desc(d);
  if (rc != SF_OK) return -rc;
  const sf::ConvArgs a = conv_args(d, d->n, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, false);
  return reads_planes(pick_stage2(d, a)) ? SF_BITMAP_PLANES : SF_BITMAP_PIXEL_MAJOR;
}

int sf_conv2d_sparse_layout(const sf_conv_desc* d, const uint32_t* bits, int32_t layout, const uint32_t* flags,
                            const void* x, const float* wt, const float* bias, void* y, void* stream) {
  if (layout != SF_BITMAP_PIXEL_MAJOR && layout != SF_BITMAP_PLANES) return fail(SF_ERR_INVALID, "unknown bitmap layout");
  int rc = check_desc(d);
  if (rc != SF_OK) return rc;
  if (d->n == 0) return SF_OK;
  if (bits == nullptr || flags == nullptr || x == nullptr || wt == nullptr || y == nullptr)
    return fail(SF_ERR_INVALID, "NULL pointer");
  sf::ConvArgs a = conv_args(d, d->n, bits, flags, x, wt, bias, y, false);
  const Stage2 k = pick_stage2(d, a);
  // With one word per pixel the two layouts are the same words.
  if (layout == SF_BITMAP_PLANES && a.cwp > 1) {
    if (!reads_planes(k)) return fail(SF_ERR_UNSUPPORTED, "word planes: this shape's Stage 2 reads pixel-major words");
    use_planes(a);
  }
  return run_stage2(k, d, a, stream);
}

// ---- sparse linear ------------------------------------------------------------

size_t sf_linear_bitmap_bytes(int64_t m, int32_t k) {
  if (m <= 0 || k < 1) return 0;
  return (size_t)m * (size_t)sf::linear_words_per_row(k) * 4u;
}

size_t sf_linear_flags_bytes(int64_t m) {
  if (m <= 0) return 0;
  return (size_t)((m + sf::kLinearRowChunk - 1) / sf::kLinearRowChunk) * 4u;
}

size_t sf_linear_workspace_size(int64_t m, int32_t k) {
  if (m <= 0 || k < 1) return 0;
  return align256(sf_linear_bitmap_bytes(m, k)) + align256(sf_linear_flags_bytes(m));
}

int sf_linear_prescan(const void* x, int32_t dtype, int64_t m, int32_t k, float threshold, uint32_t* bits,
                      uint32_t* flags, void* stream) {
  if (m < 0 || k < 1) return fail(SF_ERR_INVALID, "bad linear prescan shape");
  if (!dtype_ok(dtype)) return fail(SF_ERR_INVALID, "unknown dtype");
  if (m >= (1ll << 30)) return fail(SF_ERR_UNSUPPORTED, "m >= 2^30 rows");
  if (m == 0) return SF_OK;
  if (x == nullptr || bits == nullptr || flags == nullptr) return fail(SF_ERR_INVALID, "NULL pointer");
  sf::PackArgs a{};
  a.x = x;
  a.bits = bits;
  a.flags = flags;
  a.n = m;
  a.c = k;
  a.cwp = sf::linear_words_per_row(k);
  a.total_chunks = (m + sf::kLinearRowChunk - 1) / sf::kLinearRowChunk;
  a.cutoff = sf_activity_cutoff(threshold);
  const int rc = sf::launch_pack_rows(a, dtype, static_cast<hipStream_t>(stream));
  if (rc != hipSuccess) return hip_fail(rc, "prescan_rows launch");
  return SF_OK;
}

int sf_linear_sparse(const uint32_t* bits, const uint32_t* flags, const void* x, int32_t in_dtype, int64_t m,
                     int32_t k, const float* wt, const float* bias, int32_t c_out, void* y, int32_t out_dtype,
                     void* stream) {
  if (m < 0 || k < 1 || c_out < 1) return fail(SF_ERR_INVALID, "bad linear shape");
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(SF_ERR_INVALID, "unknown dtype");
  if (out_dtype != in_dtype && out_dtype != SF_F32)
    return fail(SF_ERR_UNSUPPORTED, "out_dtype must equal in_dtype or be f32");
  if (c_out % 4 != 0) return fail(SF_ERR_UNSUPPORTED, "c_out must be a multiple of 4");
  if (m >= (1ll << 30)) return fail(SF_ERR_UNSUPPORTED, "m >= 2^30 rows");
  if (m == 0) return SF_OK;
  if (bits == nullptr || flags == nullptr || x == nullptr || wt == nullptr || y == nullptr)
    return fail(SF_ERR_INVALID, "NULL pointer");
  sf::ConvArgs a{};
  a.bits = bits;
  a.flags = flags;
  a.x = x;
  a.wt = wt;
  a.bias = bias;
  a.y = y;
  a.n = 1;
  a.c_in = k;
  a.h_in = a.h_out = (int)m;
  a.w_in = a.w_out = 1;
  a.hw_in = a.hw_out = (int)m;
  a.c_out = c_out;
  a.k = 1;
  a.s = 1;
  a.cwp = sf::linear_words_per_row(k);
  a.chunk = sf::kLinearRowChunk;
  a.chunks_per_frame = (m + sf::kLinearRowChunk - 1) / sf::kLinearRowChunk;
  a.T = 1;
  const int rc = sf::launch_linear_flat(a, in_dtype, out_dtype, static_cast<hipStream_t>(stream));
  if (rc != hipSuccess) return hip_fail(rc, "linear_flat launch");
  return SF_OK;
}

int sf_linear_mfma(const void* x, int32_t in_dtype, int64_t m, int32_t k, const uint16_t* w_hi, const uint16_t* w_lo,
                   int32_t kp, const float* bias, int32_t c_out, float threshold, void* y, int32_t out_dtype,
                   void* stream) {
  if (m < 0 || k < 1 || c_out < 1) return fail(SF_ERR_INVALID, "bad linear shape");
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(SF_ERR_INVALID, "unknown dtype");
  if (out_dtype != in_dtype && out_dtype != SF_F32)
    return fail(SF_ERR_UNSUPPORTED, "out_dtype must equal in_dtype or be f32");
  if (kp % 32 != 0 || kp < k || kp - k >= 32) return fail(SF_ERR_INVALID, "kp must be k rounded up to a multiple of 32");
  if (kp > sf::linear_mfma_max_kp()) return fail(SF_ERR_UNSUPPORTED, "k > 8192");
  if (c_out % 4 != 0) return fail(SF_ERR_UNSUPPORTED, "c_out must be a multiple of 4");
  if (m >= (1ll << 30)) return fail(SF_ERR_UNSUPPORTED, "m >= 2^30 rows");
  if (m == 0) return SF_OK;
  if (x == nullptr || w_hi == nullptr || w_lo == nullptr || y == nullptr) return fail(SF_ERR_INVALID, "NULL pointer");
  if ((reinterpret_cast<uintptr_t>(w_hi) | reinterpret_cast<uintptr_t>(w_lo)) & 15)
    return fail(SF_ERR_INVALID, "w_hi / w_lo must be 16-byte aligned");
  sf::LinMfmaArgs a{};
  a.x = x;
  a.wh = w_hi;
  a.wl = w_lo;
  a.bias = bias;
  a.y = y;
  a.m = m;
  a.k = k;
  a.kp = kp;
  a.c_out = c_out;
  a.cutoff = sf_activity_cutoff(threshold);
  const int rc = sf::launch_linear_mfma(a, in_dtype, out_dtype, static_cast<hipStream_t>(stream));
  if (rc != hipSuccess) return hip_fail(rc, "linear_mfma launch");
  return SF_OK;
}

int sf_linear_mfma_bits(const uint32_t* bits, const uint32_t* flags, const void* x, int32_t in_dtype, int64_t m,
                        int32_t k, const uint16_t* w_hi, const uint16_t* w_lo, int32_t kp, const float* bias,
                        int32_t c_out, float threshold, void* y, int32_t out_dtype, void* stream) {
  if (m < 0 || k < 1 || c_out < 1) return fail(SF_ERR_INVALID, "bad linear shape");
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(SF_ERR_INVALID, "unknown dtype");
  if (out_dtype != in_dtype && out_dtype != SF_F32)
    return fail(SF_ERR_UNSUPPORTED, "out_dtype must equal in_dtype or be f32");
  if (kp % 32 != 0 || kp < k || kp - k >= 32) return fail(SF_ERR_INVALID, "kp must be k rounded up to a multiple of 32");
  if (kp > sf::linear_mfma_max_kp()) return fail(SF_ERR_UNSUPPORTED, "k > 8192");
  if (c_out % 4 != 0) return fail(SF_ERR_UNSUPPORTED, "c_out must be a multiple of 4");
  const int cwp = sf::linear_words_per_row(k);
  if (m * (int64_t)cwp * 4 >= (1ll << 31)) return fail(SF_ERR_UNSUPPORTED, "bitmap of 2^31 bytes or more");
  if (m == 0) return SF_OK;
  if (bits == nullptr || flags == nullptr || x == nullptr || w_hi == nullptr || w_lo == nullptr || y == nullptr)
    return fail(SF_ERR_INVALID, "NULL pointer");
  if ((reinterpret_cast<uintptr_t>(w_hi) | reinterpret_cast<uintptr_t>(w_lo)) & 15)
    return fail(SF_ERR_INVALID, "w_hi / w_lo must be 16-byte aligned");
  sf::LinMfmaArgs a{};
  a.x = x;
  a.wh = w_hi;
  a.wl = w_lo;
  a.bias = bias;
  a.y = y;
  a.m = m;
  a.k = k;
  a.kp = kp;
  a.c_out = c_out;
  a.cutoff = sf_activity_cutoff(threshold);
  const int rc = sf::launch_linear_bits_mfma(a, bits, flags, cwp, in_dtype, out_dtype, static_cast<hipStream_t>(stream));
  if (rc != hipSuccess) return hip_fail(rc, "linear_bits_mfma launch");
  return SF_OK;
}

int sf_linear_forward(const void* x, int32_t in_dtype, int64_t m, int32_t k, const float* wt, const float* bias,
                      int32_t c_out, float threshold, void* workspace, size_t workspace_bytes, void* y,
                      int32_t out_dtype, void* stream) {
  if (m < 0 || k < 1 || c_out < 1) return fail(SF_ERR_INVALID, "bad linear shape");
  if (m == 0) return SF_OK;
  if (workspace == nullptr) return fail(SF_ERR_INVALID, "NULL pointer");
  if (workspace_bytes < sf_linear_workspace_size(m, k)) return fail(SF_ERR_WORKSPACE, "workspace too small");
  uint32_t* bits = static_cast<uint32_t*>(workspace);
  uint32_t* flags =
      reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + align256(sf_linear_bitmap_bytes(m, k)));
  // Validate the Stage-2 arguments before the prescan is queued.
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(SF_ERR_INVALID, "unknown dtype");
  if (out_dtype != in_dtype && out_dtype != SF_F32)
    return fail(SF_ERR_UNSUPPORTED, "out_dtype must equal in_dtype or be f32");
  if (c_out % 4 != 0) return fail(SF_ERR_UNSUPPORTED, "c_out must be a multiple of 4");
  if (x == nullptr || wt == nullptr || y == nullptr) return fail(SF_ERR_INVALID, "NULL pointer");
  int rc = sf_linear_prescan(x, in_dtype, m, k, threshold, bits, flags, stream);
  if (rc != SF_OK) return rc;
  return sf_linear_sparse(bits, flags, x, in_dtype, m, k, wt, bias, c_out, y, out_dtype, stream);
}

// ---- sparse batched matmul ------------------------------------------------------

int sf_bmm_supported(int32_t k, int32_t n) { return k >= 1 && n >= 1 && sf::bmm_column_blocks(k, n) > 0; }

int sf_bmm_mfma_supported(int32_t k, int32_t n) { return sf::bmm_mfma_supported(k, n) ? 1 : 0; }

namespace {

int bmm_common(const void* a, const void* b, int32_t in_dtype, int64_t batches, int32_t m, int32_t k, int32_t n,
               int64_t b_stride_batch, int64_t b_stride_k, int64_t b_stride_n, float threshold, float alpha, void* c,
               int32_t out_dtype, void* stream, bool mfma) {
  if (batches < 0 || m < 0 || k < 1 || n < 1) return fail(SF_ERR_INVALID, "bad bmm shape");
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(SF_ERR_INVALID, "unknown dtype");
  if (out_dtype != in_dtype && out_dtype != SF_F32)
    return fail(SF_ERR_UNSUPPORTED, "out_dtype must equal in_dtype or be f32");
  if (mfma ? !sf::bmm_mfma_supported(k, n) : sf::bmm_column_blocks(k, n) == 0)
    return fail(SF_ERR_UNSUPPORTED, mfma ? "k > 256 or B's bf16 copy exceeds the 64 KB LDS budget"
                                         : "k > 252: a 64-column block of B exceeds the 64 KB LDS budget");
  if (b_stride_k < 0 || b_stride_n < 0 || b_stride_batch < 0) return fail(SF_ERR_INVALID, "negative stride");
  if (batches == 0 || m == 0) return SF_OK;
  if (a == nullptr || b == nullptr || c == nullptr) return fail(SF_ERR_INVALID, "NULL pointer");
  sf::BmmArgs args{};
  args.a = a;
  args.b = b;
  args.c = c;
  args.batches = batches;
  args.m = m;
  args.k = k;
  args.n = n;
  args.b_stride_batch = b_stride_batch;
  args.b_stride_k = b_stride_k;
  args.b_stride_n = b_stride_n;
  args.cutoff = sf_activity_cutoff(threshold);
  args.alpha = alpha;
  const int rc = mfma ? sf::launch_bmm_mfma(args, in_dtype, out_dtype, static_cast<hipStream_t>(stream))
                      : sf::launch_bmm(args, in_dtype, out_dtype, static_cast<hipStream_t>(stream));
  if (rc != hipSuccess) return hip_fail(rc, mfma ? "bmm_mfma launch" : "bmm_sparse launch");
  return SF_OK;
}

}  // namespace

int sf_bmm_mfma(const void* a, const void* b, int32_t in_dtype, int64_t batches, int32_t m, int32_t k, int32_t n,
                int64_t b_stride_batch, int64_t b_stride_k, int64_t b_stride_n, float threshold, float alpha, void* c,
                int32_t out_dtype, void* stream) {
  return bmm_common(a, b, in_dtype, batches, m, k, n, b_stride_batch, b_stride_k, b_stride_n, threshold, alpha, c,
                    out_dtype, stream, true);
}

int sf_bmm_sparse(const void* a, const void* b, int32_t in_dtype, int64_t batches, int32_t m, int32_t k, int32_t n,
                  int64_t b_stride_batch, int64_t b_stride_k, int64_t b_stride_n, float threshold, float alpha,
                  void* c, int32_t out_dtype, void* stream) {
  return bmm_common(a, b, in_dtype, batches, m, k, n, b_stride_batch, b_stride_k, b_stride_n, threshold, alpha, c,
                    out_dtype, stream, false);
}

// ---- fused spike attention ----------------------------------------------------

int sf_spike_attention_supported(int32_t s, int32_t d) {
  return s >= 1 && (d == 16 || d == 32 || d == 64) && sf::attn_lds_bytes(s, d) <= (size_t)sf::kMaxLdsBytes;
}

int sf_spike_attention(const void* q, const void* k, const void* v, int32_t in_dtype, int64_t tb, int32_t s,
                       int32_t h, int32_t d, const int64_t* qkv_strides, float scale, float threshold, void* y,
                       const int64_t* y_strides, int32_t out_dtype, void* stream) {
  if (tb < 0 || s < 1 || h < 1 || d < 1) return fail(SF_ERR_INVALID, "bad attention shape");
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(SF_ERR_INVALID, "unknown dtype");
  if (out_dtype != in_dtype && out_dtype != SF_F32)
    return fail(SF_ERR_UNSUPPORTED, "out_dtype must equal in_dtype or be f32");
  if (!sf_spike_attention_supported(s, d))
    return fail(SF_ERR_UNSUPPORTED, "head_dim must be 16, 32 or 64 and 2*s*d + d*(d+1) floats fit 160 KB of LDS");
  if (qkv_strides == nullptr || y_strides == nullptr) return fail(SF_ERR_INVALID, "NULL strides");
  if (tb == 0) return SF_OK;
  if (q == nullptr || k == nullptr || v == nullptr || y == nullptr) return fail(SF_ERR_INVALID, "NULL pointer");
  sf::AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.y = y;
  a.tb = tb;
  a.s = s;
  a.h = h;
  a.d = d;
  a.s_tb = qkv_strides[0];
  a.s_m = qkv_strides[1];
  a.s_h = qkv_strides[2];
  a.y_tb = y_strides[0];
  a.y_m = y_strides[1];
  a.y_h = y_strides[2];
  a.scale = scale;
  a.cutoff = sf_activity_cutoff(threshold);
  const int rc = sf::launch_spike_attn(a, in_dtype, out_dtype, static_cast<hipStream_t>(stream));
  if (rc != hipSuccess) return hip_fail(rc, "spike_attention launch");
  return SF_OK;
}

int sf_conv2d_forward(const sf_conv_desc* d, const void* x, const float* wt, const float* bias, float threshold,
                      void* workspace, size_t workspace_bytes, void* y, void* stream) {
  int rc = check_desc(d);
  if (rc != SF_OK) return rc;
  if (d->n == 0) return SF_OK;
  if (x == nullptr || wt == nullptr || y == nullptr || workspace == nullptr)
    return fail(SF_ERR_INVALID, "NULL pointer");
  if (workspace_bytes < sf_conv2d_workspace_size(d)) return fail(SF_ERR_WORKSPACE, "workspace too small");
  // Small 3x3 layers on 32-wide frames: the prescan runs inside the conv
  // kernel, one launch and no bitmap in HBM.  (The matrix-core stem path
  // reads the bitmap, so it keeps the two stages.)
  {
    const sf::ConvArgs fa = conv_args(d, d->n, nullptr, nullptr, x, wt, bias, y, false);
    if (!(d->in_dtype == SF_F32 && sf::mfma_conv_applicable(fa)) && sf::rows_fused_applicable(fa)) {
      rc = sf::launch_conv_rows_fused(fa, d->in_dtype, d->out_dtype, sf_activity_cutoff(threshold),
                                      static_cast<hipStream_t>(stream));
      if (rc != hipSuccess) return hip_fail(rc, "conv_rows_fused launch");
      return SF_OK;
    }
  }
  const Workspace ws = carve(workspace, d->n, d->c_in, d->h_in, d->w_in);
  sf::ConvArgs a = conv_args(d, d->n, ws.bits, ws.flags, x, wt, bias, y, false);
  const Stage2 k = pick_stage2(d, a);
  const bool planar = reads_planes(k);
  rc = prescan_for(d, d->n, x, threshold, planar, ws.bits, ws.flags, stream);
  if (rc != SF_OK) return rc;
  if (planar) use_planes(a);
  return run_stage2(k, d, a, stream);
}

}  // extern "C"

// ---- no-allocation variant of sf_conv2d_forward -------------------------------
// The bitmap and flags of sf_conv2d_forward_noalloc live in `scratch`, a fixed
// array of the library's device image: each GPU the library runs on holds its
// own copy (allocated when the code object is loaded there) until the process
// ends.  In host code the symbol is only a stand-in: its device address is
// looked up once per GPU with hipGetSymbolAddress (with that GPU current) and
// only that address reaches a kernel.  k_pack writes every bitmap word and
// every flag of the frames it covers, so the previous call's contents need no
// clearing.  The first call on a GPU does these lookups (the scratch and the
// dense-tile queue), which may load the library's code objects there; later
// calls only launch.
static __device__ __align__(256) uint32_t scratch[SF_NOALLOC_SCRATCH_BYTES / 4];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail((int)e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(SF_ERR_UNSUPPORTED, "device index out of range for the scratch table");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail((int)e, "hipGetSymbolAddress(scratch)");
    if (p == nullptr) return fail(SF_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    // The dense-tile queue of the 3x3 pixel-tile kernels is library device
    // memory too: look it up now, with the scratch, so that no later call
    // on this GPU does a lookup (which may load a code object).
    e = (hipError_t)sf::dense_queue_prepare();
    if (e != hipSuccess) return hip_fail((int)e, "dense-tile queue lookup");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SF_OK;
}

}  // namespace

extern "C" {

int sf_conv2d_forward_noalloc(const sf_conv_desc* d, const void* x, const float* wt, const float* bias,
                              float threshold, void* y, void* stream) {
  int rc = check_desc(d);
  if (rc != SF_OK) return rc;
  if (d->n == 0) return SF_OK;
  if (x == nullptr || wt == nullptr || y == nullptr) return fail(SF_ERR_INVALID, "NULL pointer");
  const size_t need = sf_conv2d_workspace_size(d);
  if (need > (size_t)SF_NOALLOC_SCRATCH_BYTES)
    return fail(SF_ERR_WORKSPACE, "sf_conv2d_forward_noalloc: the bitmap of these frames needs " +
                                      std::to_string(need) + " bytes; the library scratch holds " +
                                      std::to_string((size_t)SF_NOALLOC_SCRATCH_BYTES) +
                                      " per GPU (split the frames over several calls, or pass a workspace to "
                                      "sf_conv2d_forward)");
  void* ws = nullptr;
  rc = scratch_of_current_device(&ws);
  if (rc != SF_OK) return rc;
  return sf_conv2d_forward(d, x, wt, bias, threshold, ws, need, y, stream);
}

int sf_conv_lif_forward(const sf_conv_desc* d, int32_t T, const void* x, const float* wt, const float* bias,
                        const sf_lif_params* lif, float threshold, const float* v_init, void* spikes, float* v_out,
                        void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_desc(d, false);
  if (rc != SF_OK) return rc;
  if (d->stride != 1) return fail(SF_ERR_UNSUPPORTED, "fused conv-LIF supports stride 1");
  if (lif == nullptr) return fail(SF_ERR_INVALID, "lif params NULL");
  if (T < 1) return fail(SF_ERR_INVALID, "T < 1");
  if (!(lif->tau != 0.f)) return fail(SF_ERR_INVALID, "tau must be non-zero");
  if (d->n == 0) return SF_OK;
  if (x == nullptr || wt == nullptr || spikes == nullptr || v_out == nullptr || workspace == nullptr)
    return fail(SF_ERR_INVALID, "NULL pointer");
  if (workspace_bytes < sf_conv_lif_workspace_size(d, T)) return fail(SF_ERR_WORKSPACE, "workspace too small");
  const int64_t frames = d->n * (int64_t)T;
  const Workspace ws = carve(workspace, frames, d->c_in, d->h_in, d->w_in);
  // Flags/chunks are indexed by frame t*N + n over all T*N frames.
  sf::ConvArgs a = conv_args(d, frames, ws.bits, ws.flags, x, wt, bias, spikes, true);
  const bool planar = sf::px3_applicable(a);
  rc = prescan_for(d, frames, x, threshold, planar, ws.bits, ws.flags, stream);
  if (rc != SF_OK) return rc;
  if (planar) use_planes(a);
  a.total_groups = d->n * (int64_t)a.groups_per_frame;
  a.v_out = v_out;
  a.v_init = v_init;
  a.T = T;
  a.tau = lif->tau;
  a.v_th = lif->v_threshold;
  a.v_reset = lif->v_reset;
  a.hard_reset = lif->hard_reset != 0;
  a.decay_input = lif->decay_input != 0;
  if (sf::px3_applicable(a)) {
    rc = sf::launch_conv_lif_px3(a, d->in_dtype, d->out_dtype, static_cast<hipStream_t>(stream));
    if (rc != hipSuccess) return hip_fail(rc, "conv_lif_px3 launch");
    return SF_OK;
  }
  rc = sf::launch_conv_lif(a, d->in_dtype, d->out_dtype, static_cast<hipStream_t>(stream));
  if (rc != hipSuccess) return hip_fail(rc, "conv_lif launch");
  return SF_OK;
}

static int conv1x1_lif_impl(const sf_conv_desc* d, int32_t T, const uint32_t* bits, const uint32_t* flags,
                            const void* x, const float* wt, const float* bias, const void* x2,
                            const uint32_t* res_bits, const sf_lif_params* lif, const float* v_init, void* spikes,
                            float* v_out, uint32_t* out_bits, uint32_t* out_flags, int32_t out_layout,
                            void* stream) {
  if (out_layout != SF_BITMAP_PIXEL_MAJOR && out_layout != SF_BITMAP_PLANES)
    return fail(SF_ERR_INVALID, "unknown bitmap layout");
  int rc = check_desc(d, false);
  if (rc != SF_OK) return rc;
  if (d->kernel != 1 || d->stride != 1) return fail(SF_ERR_UNSUPPORTED, "fused conv1x1-LIF: 1x1 stride 1 only");
  if (d->c_out % 4 != 0) return fail(SF_ERR_UNSUPPORTED, "c_out must be a multiple of 4");
  if (lif == nullptr) return fail(SF_ERR_INVALID, "lif params NULL");
  if (T < 1) return fail(SF_ERR_INVALID, "T < 1");
  if (!(lif->tau != 0.f)) return fail(SF_ERR_INVALID, "tau must be non-zero");
  if ((out_bits == nullptr) != (out_flags == nullptr)) return fail(SF_ERR_INVALID, "out_bits and out_flags go together");
  if (out_bits != nullptr && sf::words_per_pixel(d->c_out) > 64) return fail(SF_ERR_UNSUPPORTED, "c_out > 2048");
  if (d->n == 0) return SF_OK;
  if (bits == nullptr || flags == nullptr || x == nullptr || wt == nullptr || spikes == nullptr || v_out == nullptr)
    return fail(SF_ERR_INVALID, "NULL pointer");
  const int64_t frames = d->n * (int64_t)T;
  sf::ConvArgs a = conv_args(d, frames, bits, flags, x, wt, bias, spikes, true);
  a.v_out = v_out;
  a.v_init = v_init;
  a.T = T;
  a.tau = lif->tau;
  a.v_th = lif->v_threshold;
  a.v_reset = lif->v_reset;
  a.hard_reset = lif->hard_reset != 0;
  a.decay_input = lif->decay_input != 0;
  const sf::PackPlan op = sf::make_pack_plan(frames, d->c_out, d->h_out, d->w_out);
  rc = sf::launch_conv_lif_flat(a, d->in_dtype, d->out_dtype, x2, res_bits, out_bits, out_flags, op.cwp,
                                out_layout == SF_BITMAP_PLANES ? 1 : 0, op.chunk, op.chunks_per_frame,
                                static_cast<hipStream_t>(stream));
  if (rc != hipSuccess) return hip_fail(rc, "conv_lif_flat launch");
  return SF_OK;
}

int sf_conv1x1_lif_sparse(const sf_conv_desc* d, int32_t T, const uint32_t* bits, const uint32_t* flags, const void* x,
                          const float* wt, const float* bias, const void* x2, const sf_lif_params* lif,
                          const float* v_init, void* spikes, float* v_out, uint32_t* out_bits, uint32_t* out_flags,
                          void* stream) {
  return conv1x1_lif_impl(d, T, bits, flags, x, wt, bias, x2, nullptr, lif, v_init, spikes, v_out, out_bits,
                          out_flags, SF_BITMAP_PIXEL_MAJOR, stream);
}

int sf_conv1x1_lif_sparse_layout(const sf_conv_desc* d, int32_t T, const uint32_t* bits, const uint32_t* flags,
                                 const void* x, const float* wt, const float* bias, const void* x2,
                                 const sf_lif_params* lif, const float* v_init, void* spikes, float* v_out,
                                 uint32_t* out_bits, uint32_t* out_flags, int32_t out_layout, void* stream) {
  return conv1x1_lif_impl(d, T, bits, flags, x, wt, bias, x2, nullptr, lif, v_init, spikes, v_out, out_bits,
                          out_flags, out_layout, stream);
}

int sf_conv1x1_lif_sparse_binres(const sf_conv_desc* d, int32_t T, const uint32_t* bits, const uint32_t* flags,
                                 const void* x, const float* wt, const float* bias, const uint32_t* res_bits,
                                 const sf_lif_params* lif, const float* v_init, void* spikes, float* v_out,
                                 uint32_t* out_bits, uint32_t* out_flags, void* stream) {
  if (d != nullptr && d->n > 0 && res_bits == nullptr) return fail(SF_ERR_INVALID, "res_bits NULL");
  return conv1x1_lif_impl(d, T, bits, flags, x, wt, bias, nullptr, res_bits, lif, v_init, spikes, v_out, out_bits,
                          out_flags, SF_BITMAP_PIXEL_MAJOR, stream);
}

int sf_spike_maxpool2d(const uint32_t* bits, int64_t n, int32_t c, int32_t h_in, int32_t w_in, int32_t k,
                       int32_t stride, int32_t padding, void* y, int32_t out_dtype, uint32_t* out_bits,
                       void* stream) {
  if (!dtype_ok(out_dtype)) return fail(SF_ERR_INVALID, "unknown dtype");
  if (n < 0 || c < 0 || h_in < 0 || w_in < 0) return fail(SF_ERR_INVALID, "negative size");
  if (k < 1 || stride < 1 || padding < 0 || 2 * padding > k)
    return fail(SF_ERR_INVALID, "kernel >= 1, stride >= 1, 0 <= padding <= kernel / 2");
  if (c > 32 * sf::kSpikePoolMaxWords) return fail(SF_ERR_UNSUPPORTED, "spike max pooling: c <= 256");
  if ((int64_t)h_in * w_in > INT32_MAX) return fail(SF_ERR_UNSUPPORTED, "h_in * w_in < 2^31");
  const int h_out = h_in + 2 * padding < k ? 0 : (h_in + 2 * padding - k) / stride + 1;
  const int w_out = w_in + 2 * padding < k ? 0 : (w_in + 2 * padding - k) / stride + 1;
  if (n == 0 || c == 0 || h_out == 0 || w_out == 0) return SF_OK;
  if (bits == nullptr || y == nullptr || out_bits == nullptr) return fail(SF_ERR_INVALID, "NULL pointer");
  const int cwp = sf::words_per_pixel(c);
  if (cwp > sf::kSpikePoolMaxWords) return fail(SF_ERR_UNSUPPORTED, "spike max pooling: c <= 256");
  const int rc = sf::launch_spike_maxpool(bits, n, c, h_in, w_in, h_out, w_out, k, stride, padding, cwp, out_dtype,
                                          y, out_bits, static_cast<hipStream_t>(stream));
  return rc == (int)hipSuccess ? SF_OK : fail(SF_ERR_HIP, hipGetErrorString((hipError_t)rc));
}

int sf_lif_multistep(const void* x, const void* x2, int32_t in_dtype, int32_t T, int64_t n, int32_t c, int64_t hw,
                     const sf_lif_params* lif, const float* v_init, void* spikes, int32_t out_dtype, float* v_out,
                     uint32_t* bits, uint32_t* flags, void* stream) {
  return sf_lif_multistep_layout(x, x2, in_dtype, T, n, c, hw, lif, v_init, spikes, out_dtype, v_out, bits, flags,
                                 SF_BITMAP_PIXEL_MAJOR, stream);
}

int sf_lif_multistep_layout(const void* x, const void* x2, int32_t in_dtype, int32_t T, int64_t n, int32_t c,
                            int64_t hw, const sf_lif_params* lif, const float* v_init, void* spikes, int32_t out_dtype,
                            float* v_out, uint32_t* bits, uint32_t* flags, int32_t bits_layout, void* stream) {
  if (bits_layout != SF_BITMAP_PIXEL_MAJOR && bits_layout != SF_BITMAP_PLANES)
    return fail(SF_ERR_INVALID, "unknown bitmap layout");
  if (lif == nullptr) return fail(SF_ERR_INVALID, "lif params NULL");
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(SF_ERR_INVALID, "unknown dtype");
  if (out_dtype != in_dtype && out_dtype != SF_F32)
    return fail(SF_ERR_UNSUPPORTED, "out_dtype must equal in_dtype or be f32");
  if (T < 1 || n < 0 || c < 0 || hw < 0) return fail(SF_ERR_INVALID, "T < 1 or negative size");
  if (!(lif->tau != 0.f)) return fail(SF_ERR_INVALID, "tau must be non-zero");
  if ((bits == nullptr) != (flags == nullptr)) return fail(SF_ERR_INVALID, "bits and flags go together");
  if (bits != nullptr && (hw > INT32_MAX || c > 4096)) return fail(SF_ERR_UNSUPPORTED, "spike map: c <= 4096, hw < 2^31");
  if (n == 0 || c == 0 || hw == 0) return SF_OK;
  if (x == nullptr || spikes == nullptr || v_out == nullptr) return fail(SF_ERR_INVALID, "NULL pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int cwp = 0;
  int64_t nflags = 0;
  if (bits != nullptr) {
    // The spike map of T*n frames of c x hw, exactly as sf_prescan_pack lays
    // it out; every chunk is binary, so the flags are all zero.
    const sf::PackPlan pl = sf::make_pack_plan((int64_t)T * n, c, 1, (int)hw);
    cwp = pl.cwp;
    nflags = pl.total_chunks;
  }
  const int rc = sf::launch_lif_multistep(x, x2, in_dtype, T, n, c, hw, lif->tau, lif->v_threshold, lif->v_reset,
                                          lif->hard_reset, lif->decay_input, v_init, spikes, out_dtype, v_out, bits, cwp,
                                          bits_layout == SF_BITMAP_PLANES ? 1 : 0, flags, nflags, s);
  if (rc != hipSuccess) return hip_fail(rc, "lif_multistep launch");
  return SF_OK;
}

int sf_timing_enable(int32_t enable) {
  std::lock_guard<std::mutex> lk(g_tmu);
  g_timing = enable != 0;
  return SF_OK;
}

int sf_timing_collect(void) {
  std::vector<TimingRec> recs;
  {
    std::lock_guard<std::mutex> lk(g_tmu);
    recs.swap(g_pending);
  }
  int status = SF_OK;
  for (auto& r : recs) {
    if (r.end != nullptr && r.start != nullptr) {
      if (hipEventSynchronize(r.end) == hipSuccess) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, r.start, r.end) == hipSuccess) {
          std::lock_guard<std::mutex> lk(g_tmu);
          g_total_ms[r.id] += ms;
          g_count[r.id] += 1;
        } else {
          status = SF_ERR_HIP;
        }
      } else {
        status = SF_ERR_HIP;
      }
    }
    if (r.start) (void)hipEventDestroy(r.start);
    if (r.end) (void)hipEventDestroy(r.end);
  }
  return status;
}

int64_t sf_timing_query(const char* kernel, double* total_ms) {
  std::lock_guard<std::mutex> lk(g_tmu);
  for (int i = 0; i < sf::K_COUNT; ++i) {
    if (kernel != nullptr && strcmp(kernel, g_names[i]) == 0) {
      if (total_ms) *total_ms = g_total_ms[i];
      return g_count[i];
    }
  }
  if (total_ms) *total_ms = 0.0;
  return -1;
}

void sf_timing_reset(void) {
  std::lock_guard<std::mutex> lk(g_tmu);
  for (int i = 0; i < sf::K_COUNT; ++i) {
    g_total_ms[i] = 0.0;
    g_count[i] = 0;
  }
}

}  // extern "C"
