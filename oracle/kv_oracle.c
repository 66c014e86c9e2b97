/*
 * kv_oracle.c -- CPU restatement of DaseR's KV save/load copy path, plus the
 * textbook RoPE re-rotation the load path adds.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker for libdaser_kv's HIP
 * kernels: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it. No product code path calls it.
 *
 * Parity pins (each function is checked by tests/test_oracle.py):
 *   orc_gather / orc_scatter    against a brute-force per-byte restatement of
 *       the reference loops (bytes(kv[:, b]) at i*SLOT + l*LAYER), the
 *       reference's slot-size constants, and the round-trip identity;
 *   orc_decode / orc_encode     against torch's bfloat16 / float16 /
 *       float8_e4m3fn / float8_e5m2 conversions (all 256 codes of each 8-bit
 *       format, sweeps of fp32 values);
 *   orc_scatter_rerotate        against closed forms: zero delta is a copy,
 *       R(a)R(-a) = I, R(a)R(b) = R(a+b), pair norms preserved, the complex
 *       multiplication (x1 + i x2) e^{i delta w_j}, and single-pair known
 *       answers (cos d, sin d).
 *
 * Layouts are those of include/daser_kv.h. Pointers here are host pointers.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define ORC_BF16 0
#define ORC_FP16 1
#define ORC_E4M3 2
#define ORC_E5M2 3
#define ORC_IS_FP8(d) ((d) == ORC_E4M3 || (d) == ORC_E5M2)

#define ORC_NEOX 0
#define ORC_GPTJ 1

/* ---- save: reference daser/connector/daser_connector.py:610-632 ----------
 * for each page p (request r, slot i, block b = block_ids[i]) and layer l:
 *   staging[dst_off : dst_off + nbytes] = bytes(kv_l[:, b])
 * with dst_off = slot_offsets[p] + l * LAYER and bytes(kv_l[:, b]) the K page
 * followed by the V page (C order of kv_l[:, b], shape (2, bs, H, D)). */
void orc_gather(const uint8_t* const* layer_base, int n_layers,
                int64_t kv_stride, int64_t page_stride, int64_t page_bytes,
                const int32_t* page_ids, const int64_t* slot_offsets,
                int n_pages, uint8_t* staging, int64_t layer_bytes,
                int layer0) {
  for (int p = 0; p < n_pages; ++p) {
    for (int l = 0; l < n_layers; ++l) {
      const uint8_t* src = layer_base[l] + (int64_t)page_ids[p] * page_stride;
      uint8_t* dst = staging + slot_offsets[p] + (int64_t)(layer0 + l) * layer_bytes;
      memcpy(dst, src, (size_t)page_bytes);
      memcpy(dst + page_bytes, src + kv_stride, (size_t)page_bytes);
    }
  }
}

/* ---- load: reference daser/connector/daser_connector.py:536-551 ----------
 * kv_l[:, b].copy_(staging[off : off + nbytes].view(dtype).view(shape)) */
void orc_scatter(uint8_t* const* layer_base, int n_layers, int64_t kv_stride,
                 int64_t page_stride, int64_t page_bytes,
                 const int32_t* page_ids, const int64_t* slot_offsets,
                 int n_pages, const uint8_t* staging, int64_t layer_bytes,
                 int layer0) {
  for (int p = 0; p < n_pages; ++p) {
    for (int l = 0; l < n_layers; ++l) {
      uint8_t* dst = layer_base[l] + (int64_t)page_ids[p] * page_stride;
      const uint8_t* src = staging + slot_offsets[p] + (int64_t)(layer0 + l) * layer_bytes;
      memcpy(dst, src, (size_t)page_bytes);
      memcpy(dst + kv_stride, src + page_bytes, (size_t)page_bytes);
    }
  }
}

/* ---- element formats, from their specifications -------------------------
 * bf16: IEEE binary32 truncated to 1+8+7 bits.
 * fp16: IEEE binary16, 1+5+10, bias 15.
 * e4m3: OCP 8-bit float e4m3fn, 1+4+3, bias 7, no infinities, only
 *       S.1111.111 is NaN, max finite 448.
 * e5m2: OCP 8-bit float e5m2, 1+5+2, bias 15, IEEE-style infinities
 *       (S.11111.00) and NaNs (S.11111.{01,10,11}), max finite 57344. */
typedef struct {
  int mbits, emin, bias, sign_shift;
  double maxv;
} fmt_t;

static const fmt_t FMT[4] = {
    {7, -126, 127, 15, 3.38953138925153547590470800371487866880e38},
    {10, -14, 15, 15, 65504.0},
    {3, -6, 7, 7, 448.0},
    {2, -14, 15, 7, 57344.0},
};

double orc_decode(int dtype, uint32_t bits) {
  const fmt_t* f = &FMT[dtype];
  const int ebits = f->sign_shift - f->mbits;
  const uint32_t emask = (1u << ebits) - 1u;
  const uint32_t s = (bits >> f->sign_shift) & 1u;
  const uint32_t E = (bits >> f->mbits) & emask;
  const uint32_t M = bits & ((1u << f->mbits) - 1u);
  double v;
  if (dtype == ORC_E4M3) {
    if (E == 15 && M == 7) return NAN;
  } else if (E == emask) {
    if (M) return NAN;
    return s ? -INFINITY : INFINITY;
  }
  if (E == 0)
    v = ldexp((double)M, f->emin - f->mbits);
  else
    v = ldexp(1.0 + ldexp((double)M, -f->mbits), (int)E - f->bias);
  return s ? -v : v;
}

/* Rounds v to the format (round to nearest, ties to even, at the format's
 * precision and subnormal spacing) and returns its bit pattern.
 * The 8-bit formats saturate to +-max (448, 57344) before rounding, so they
 * never overflow (e5m2 infinities included, as a saturating conversion
 * does); bf16/fp16 overflow to infinity. NaN -> 0x7FC0 / 0x7E00 / 0x7F. */
uint32_t orc_encode(int dtype, double v) {
  const fmt_t* f = &FMT[dtype];
  if (isnan(v)) return dtype == ORC_BF16 ? 0x7fc0u : dtype == ORC_FP16 ? 0x7e00u : 0x7fu;
  if (ORC_IS_FP8(dtype)) {
    if (v > f->maxv) v = f->maxv;
    if (v < -f->maxv) v = -f->maxv;
  }
  const uint32_t s = signbit(v) ? 1u : 0u;
  double a = fabs(v);
  const int ebits = f->sign_shift - f->mbits;
  if (isinf(a)) return (s << f->sign_shift) | (((1u << ebits) - 1u) << f->mbits);
  if (a == 0.0) return s << f->sign_shift;
  int e;
  frexp(a, &e);
  int ex = e - 1; /* a in [2^ex, 2^(ex+1)) */
  if (ex < f->emin) ex = f->emin;
  const double q = ldexp(1.0, ex - f->mbits);
  double r = nearbyint(a / q) * q; /* a / q is exact (power-of-two scale) */
  if (r > f->maxv) /* rounds past the largest finite value */
    return (s << f->sign_shift) | (((1u << ebits) - 1u) << f->mbits);
  if (r == 0.0) return s << f->sign_shift;
  frexp(r, &e);
  ex = e - 1;
  uint32_t E, M;
  if (ex < f->emin) {
    E = 0;
    M = (uint32_t)ldexp(r, f->mbits - f->emin);
  } else {
    E = (uint32_t)(ex + f->bias);
    M = (uint32_t)(ldexp(r, f->mbits - ex)) - (1u << f->mbits);
  }
  return (s << f->sign_shift) | (E << f->mbits) | M;
}

static uint32_t load_elem(const uint8_t* row, int dtype, int j) {
  if (ORC_IS_FP8(dtype)) return row[j];
  uint16_t h;
  memcpy(&h, row + 2 * j, 2);
  return h;
}

static void store_elem(uint8_t* row, int dtype, int j, uint32_t bits) {
  if (ORC_IS_FP8(dtype)) {
    row[j] = (uint8_t)bits;
  } else {
    uint16_t h = (uint16_t)bits;
    memcpy(row + 2 * j, &h, 2);
  }
}

/* Rotates (x1, x2) by angle a: (x1 cos a - x2 sin a, x2 cos a + x1 sin a). */
static void rot(double* x1, double* x2, double a) {
  const double c = cos(a), s = sin(a);
  const double y1 = *x1 * c - *x2 * s;
  const double y2 = *x2 * c + *x1 * s;
  *x1 = y1;
  *x2 = y2;
}

/* ---- load with re-rotation (net-new; the reference only carries the
 * integer offset, daser/position/fixed_offset.py:26-50) ---------------------
 * Scatter as orc_scatter. For a page with rotate[p] != 0, each K row (token
 * t of the page, head h) moves from its stored position stored_pos[p] + t to
 * new_pos[p] + t: x <- R(new + t) R(stored + t)^-1 x = R(delta) x with the
 * exact integer delta = (new + t) - (stored + t), evaluated as one float64
 * rotation of pair j by angle delta * w_j, w_j = inv_freq[j] if given, else
 * theta^(-2j/rot_dim). (Rotating back and then forward in two float64 steps
 * is the same map for finite inputs, but turns an infinite element into NaN
 * through inf * sin(0) when a position is 0.)
 * Pairs: neox (j, j + rot_dim/2); gptj (2j, 2j + 1). Elements >= rot_dim and
 * V are copied. e4m3 / e5m2: x = decode(q) * k_scale[layer], result /
 * k_scale is encoded (saturating). The result is rounded once to the storage format. */
void orc_scatter_rerotate(uint8_t* const* layer_base, int n_layers,
                          int64_t kv_stride, int64_t page_stride,
                          int64_t page_bytes, const int32_t* page_ids,
                          const int64_t* slot_offsets, int n_pages,
                          const uint8_t* staging, int64_t layer_bytes,
                          int layer0, int num_heads, int head_dim, int rot_dim,
                          int style, int dtype, const float* k_scale,
                          const int64_t* stored_pos, const int64_t* new_pos,
                          const int8_t* rotate, double theta,
                          const double* inv_freq) {
  const int esize = ORC_IS_FP8(dtype) ? 1 : 2;
  const int64_t row_bytes = (int64_t)head_dim * esize;
  const int64_t rows = page_bytes / row_bytes;
  const int half = rot_dim / 2;
  double w[1024];
  for (int j = 0; j < half; ++j)
    w[j] = inv_freq ? inv_freq[j] : pow(theta, -2.0 * j / rot_dim);
  orc_scatter(layer_base, n_layers, kv_stride, page_stride, page_bytes, page_ids,
              slot_offsets, n_pages, staging, layer_bytes, layer0);
  double x[2048];
  for (int p = 0; p < n_pages; ++p) {
    if (!rotate[p]) continue;
    for (int l = 0; l < n_layers; ++l) {
      const double sc = ORC_IS_FP8(dtype) ? (double)k_scale[layer0 + l] : 1.0;
      uint8_t* dst = layer_base[l] + (int64_t)page_ids[p] * page_stride;
      const uint8_t* src = staging + slot_offsets[p] + (int64_t)(layer0 + l) * layer_bytes;
      for (int64_t r = 0; r < rows; ++r) {
        const int64_t tok = r / num_heads;
        const uint8_t* srow = src + r * row_bytes;
        uint8_t* drow = dst + r * row_bytes;
        for (int j = 0; j < rot_dim; ++j) x[j] = orc_decode(dtype, load_elem(srow, dtype, j)) * sc;
        const double delta = (double)((new_pos[p] + tok) - (stored_pos[p] + tok));
        for (int j = 0; j < half; ++j) {
          double *a, *b;
          if (style == ORC_NEOX) {
            a = &x[j];
            b = &x[j + half];
          } else {
            a = &x[2 * j];
            b = &x[2 * j + 1];
          }
          rot(a, b, delta * w[j]);
        }
        for (int j = 0; j < rot_dim; ++j) store_elem(drow, dtype, j, orc_encode(dtype, x[j] / sc));
      }
    }
  }
}

/* Array forms of orc_decode / orc_encode for the Python checker. */
void orc_decode_array(int dtype, const uint32_t* bits, double* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_decode(dtype, bits[i]);
}

void orc_encode_array(int dtype, const double* v, uint32_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_encode(dtype, v[i]);
}

/* ---- token-granular forms (vLLM slot_mapping) ------------------------------
 * Token t with slot = slot_mapping[t] >= 0: its K row (row_bytes, all heads)
 * sits at layer_base[l] + (slot / bs) * page_stride + (slot % bs) * row_bytes
 * and V at + kv_stride; its record rows at staging + row_offsets[t] +
 * (layer0 + l) * layer_bytes and + page_bytes. Padding tokens (slot < 0) are
 * skipped. Per-token form of daser_connector.py:625-632 / :536-551. */
void orc_gather_slots(const uint8_t* const* layer_base, int n_layers, int64_t kv_stride,
                      int64_t page_stride, int64_t page_bytes, int block_size,
                      int64_t row_bytes, const int64_t* slot_mapping,
                      const int64_t* row_offsets, int n_tokens, uint8_t* staging,
                      int64_t layer_bytes, int layer0) {
  for (int t = 0; t < n_tokens; ++t) {
    const int64_t slot = slot_mapping[t];
    if (slot < 0) continue;
    for (int l = 0; l < n_layers; ++l) {
      const uint8_t* src = layer_base[l] + (slot / block_size) * page_stride +
                           (slot % block_size) * row_bytes;
      uint8_t* dst = staging + row_offsets[t] + (int64_t)(layer0 + l) * layer_bytes;
      memcpy(dst, src, (size_t)row_bytes);
      memcpy(dst + page_bytes, src + kv_stride, (size_t)row_bytes);
    }
  }
}

void orc_scatter_slots(uint8_t* const* layer_base, int n_layers, int64_t kv_stride,
                       int64_t page_stride, int64_t page_bytes, int block_size,
                       int64_t row_bytes, const int64_t* slot_mapping,
                       const int64_t* row_offsets, int n_tokens, const uint8_t* staging,
                       int64_t layer_bytes, int layer0) {
  for (int t = 0; t < n_tokens; ++t) {
    const int64_t slot = slot_mapping[t];
    if (slot < 0) continue;
    for (int l = 0; l < n_layers; ++l) {
      uint8_t* dst = layer_base[l] + (slot / block_size) * page_stride +
                     (slot % block_size) * row_bytes;
      const uint8_t* src = staging + row_offsets[t] + (int64_t)(layer0 + l) * layer_bytes;
      memcpy(dst, src, (size_t)row_bytes);
      memcpy(dst + kv_stride, src + page_bytes, (size_t)row_bytes);
    }
  }
}

/* Token form of orc_scatter_rerotate: orc_scatter_slots, then for every
 * valid token t with rotate[t] != 0 each head of its K row (in every layer)
 * is rotated by delta = new_pos[t] - stored_pos[t] exactly as a page row is
 * (pairs, frequencies, scales and the one rounding of orc_scatter_rerotate).
 * Net-new like the page form; the copies follow daser_connector.py:536-551. */
void orc_scatter_slots_rerotate(uint8_t* const* layer_base, int n_layers, int64_t kv_stride,
                                int64_t page_stride, int64_t page_bytes, int block_size,
                                int64_t row_bytes, const int64_t* slot_mapping,
                                const int64_t* row_offsets, int n_tokens,
                                const uint8_t* staging, int64_t layer_bytes, int layer0,
                                int num_heads, int head_dim, int rot_dim, int style, int dtype,
                                const float* k_scale, const int64_t* stored_pos,
                                const int64_t* new_pos, const int8_t* rotate, double theta,
                                const double* inv_freq) {
  const int esize = ORC_IS_FP8(dtype) ? 1 : 2;
  const int64_t head_bytes = (int64_t)head_dim * esize;
  const int half = rot_dim / 2;
  double w[1024];
  for (int j = 0; j < half; ++j)
    w[j] = inv_freq ? inv_freq[j] : pow(theta, -2.0 * j / rot_dim);
  orc_scatter_slots(layer_base, n_layers, kv_stride, page_stride, page_bytes, block_size,
                    row_bytes, slot_mapping, row_offsets, n_tokens, staging, layer_bytes,
                    layer0);
  double x[2048];
  for (int t = 0; t < n_tokens; ++t) {
    const int64_t slot = slot_mapping[t];
    if (slot < 0 || !rotate[t]) continue;
    const double delta = (double)(new_pos[t] - stored_pos[t]);
    for (int l = 0; l < n_layers; ++l) {
      const double sc = ORC_IS_FP8(dtype) ? (double)k_scale[layer0 + l] : 1.0;
      uint8_t* drow = layer_base[l] + (slot / block_size) * page_stride +
                      (slot % block_size) * row_bytes;
      const uint8_t* srow = staging + row_offsets[t] + (int64_t)(layer0 + l) * layer_bytes;
      for (int h = 0; h < num_heads; ++h) {
        const uint8_t* s = srow + h * head_bytes;
        uint8_t* d = drow + h * head_bytes;
        for (int j = 0; j < rot_dim; ++j) x[j] = orc_decode(dtype, load_elem(s, dtype, j)) * sc;
        for (int j = 0; j < half; ++j) {
          if (style == ORC_NEOX)
            rot(&x[j], &x[j + half], delta * w[j]);
          else
            rot(&x[2 * j], &x[2 * j + 1], delta * w[j]);
        }
        for (int j = 0; j < rot_dim; ++j) store_elem(d, dtype, j, orc_encode(dtype, x[j] / sc));
      }
    }
  }
}
