/*
 * t0ref.c — CPU restatement of idle-intelligence/t0-web's t0-core path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity oracle and the "port" CPU baseline).
 * Nothing in the product (t0-web_amd/) links, loads or calls this file.
 *
 * Reference files restated here (paths relative to the reference root):
 *   crates/t0-core/src/gguf.rs      container + Q8_0/Q4_0 codec
 *   crates/t0-core/src/weights.rs   config_from_gguf_metadata, export_gguf
 *   crates/t0-core/src/config.rs    layer_types
 *   crates/t0-core/src/data.rs      TimeSeries::{from_context,from_context_batch,pad}
 *   crates/t0-core/src/scaler.rs    CausalScaler
 *   crates/t0-core/src/mask.rs      patch metadata + additive masks
 *   crates/t0-core/src/ops.rs       rmsnorm, linear, residual_block, swiglu_ffn, RoPE, mhsa, quantile_head
 *   crates/t0-core/src/model.rs     forward_tensor, forward_layer, forecast drivers, forecast_rollout
 *   crates/t0-core/src/quantile.rs  interpolate_quantiles, weighted_quantile, prob_mass
 *   crates/t0-fast/src/lib.rs       forecast_batch_rows_chunked_async (ragged rows)
 *
 * Numerics: f32 everywhere the reference is f32, f64 where it is f64 (RoPE
 * tables).  Built with -ffp-contract=off so that no multiply-add is fused
 * (Rust never contracts).  Transcendentals come from the C library, which is
 * what Rust's std calls on Linux (expf, logf, log1pf, hypotf, sinhf; pow,
 * cos, sin in f64).  Matmul summation order is this file's own (fixed,
 * thread-count independent); burn-ndarray's matrixmultiply order is not
 * restated (ulp-level differences only).
 */
#define _GNU_SOURCE
#include "t0ref.h"

#include <limits.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK 32

/* ------------------------------------------------------------------------- */
/* f16 <-> f32.  `half` 2.7.1: f16->f32 is exact; f32->f16 rounds to nearest  */
/* even, overflow to infinity, NaN quieted (gguf.rs:107,120; quant.rs:60).    */
/* ------------------------------------------------------------------------- */
float t0r_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t mant = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      int shift = 0;
      while (!(mant & 0x400u)) {
        mant <<= 1;
        shift++;
      }
      mant &= 0x3ffu;
      bits = sign | ((uint32_t)(113 - shift) << 23) | (mant << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (mant << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t t0r_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t mant = x & 0x7fffffu;
  if (exp == 0xffu) {
    if (mant) return (uint16_t)(sign | 0x7c00u | 0x0200u | (mant >> 13));
    return (uint16_t)(sign | 0x7c00u);
  }
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    /* subnormal half: value / 2^-24 = (mant|1<<23) * 2^(exp-126) */
    uint32_t m = mant | 0x800000u;
    int shift = 126 - (int)exp;
    if (exp == 0) return (uint16_t)sign; /* f32 subnormals are far below half's range */
    if (shift > 24) return (uint16_t)sign;
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)h;
}

/* ------------------------------------------------------------------------- */
/* Q8_0 / Q4_0 block codec                                                   */
/* ------------------------------------------------------------------------- */
static int block_bytes(int ty) {
  switch (ty) {
    case T0R_F32: return 4;
    case T0R_F16: return 2;
    case T0R_Q4_0: return 2 + QK / 2;
    case T0R_Q8_0: return 2 + QK;
  }
  return 0;
}

/* gguf.rs:61-70 (GgmlType::row_bytes); returns 0 for a quantized count that
 * is not a multiple of 32 (the reference asserts). */
size_t t0r_row_bytes(int ty, size_t n) {
  switch (ty) {
    case T0R_F32: return n * 4;
    case T0R_F16: return n * 2;
    case T0R_Q4_0:
    case T0R_Q8_0:
      if (n % QK) return 0;
      return (n / QK) * (size_t)block_bytes(ty);
  }
  return 0;
}

/* Rust `f as i32` saturates and maps NaN to 0. */
static int32_t rust_f32_as_i32(float f) {
  if (isnan(f)) return 0;
  if (f >= 2147483647.0f) return INT_MAX;
  if (f <= -2147483648.0f) return INT_MIN;
  return (int32_t)f;
}

/* gguf.rs:100-114 quantize_q8_0 (llama.cpp quantize_row_q8_0_ref convention) */
void t0r_quantize_q8_0(const float* x, size_t n, uint8_t* out) {
  for (size_t b = 0; b < n / QK; b++) {
    const float* blk = x + b * QK;
    float amax = 0.0f;
    for (int i = 0; i < QK; i++) amax = fmaxf(amax, fabsf(blk[i]));
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t dh = t0r_f32_to_f16(d);
    uint8_t* o = out + b * (2 + QK);
    o[0] = (uint8_t)(dh & 0xff);
    o[1] = (uint8_t)(dh >> 8);
    for (int i = 0; i < QK; i++) {
      float r = roundf(blk[i] * id); /* Rust f32::round: half away from zero */
      int8_t q;
      if (isnan(r)) {
        q = 0;
      } else {
        if (r < -128.0f) r = -128.0f;
        if (r > 127.0f) r = 127.0f;
        q = (int8_t)r;
      }
      o[2 + i] = (uint8_t)q;
    }
  }
}

/* gguf.rs:116-126 dequantize_q8_0 */
void t0r_dequantize_q8_0(const uint8_t* bytes, size_t n, float* out) {
  for (size_t b = 0; b < n / QK; b++) {
    const uint8_t* blk = bytes + b * (2 + QK);
    float d = t0r_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    for (int i = 0; i < QK; i++) out[b * QK + i] = d * (float)(int8_t)blk[2 + i];
  }
}

/* gguf.rs:133-157 quantize_q4_0 (llama.cpp quantize_row_q4_0_ref convention) */
void t0r_quantize_q4_0(const float* x, size_t n, uint8_t* out) {
  for (size_t b = 0; b < n / QK; b++) {
    const float* blk = x + b * QK;
    float amax = 0.0f, max = 0.0f;
    for (int i = 0; i < QK; i++) {
      if (fabsf(blk[i]) > amax) {
        amax = fabsf(blk[i]);
        max = blk[i];
      }
    }
    float d = max / -8.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t dh = t0r_f32_to_f16(d);
    uint8_t* o = out + b * (2 + QK / 2);
    o[0] = (uint8_t)(dh & 0xff);
    o[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < QK / 2; j++) {
      float x0 = blk[j] * id;
      float x1 = blk[j + QK / 2] * id;
      int32_t i0 = rust_f32_as_i32(floorf(x0 + 8.5f));
      int32_t i1 = rust_f32_as_i32(floorf(x1 + 8.5f));
      i0 = i0 < 0 ? 0 : (i0 > 15 ? 15 : i0);
      i1 = i1 < 0 ? 0 : (i1 > 15 ? 15 : i1);
      o[2 + j] = (uint8_t)(i0 | (i1 << 4));
    }
  }
}

/* gguf.rs:159-174 dequantize_q4_0 */
void t0r_dequantize_q4_0(const uint8_t* bytes, size_t n, float* out) {
  for (size_t b = 0; b < n / QK; b++) {
    const uint8_t* blk = bytes + b * (2 + QK / 2);
    float d = t0r_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    for (int j = 0; j < QK / 2; j++) {
      uint8_t byte = blk[2 + j];
      float lo = (float)(byte & 0x0f) - 8.0f;
      float hi = (float)(byte >> 4) - 8.0f;
      out[b * QK + j] = d * lo;
      out[b * QK + j + QK / 2] = d * hi;
    }
  }
}

/* gguf.rs:213-226 dequantize_for */
int t0r_dequantize_for(int ty, const uint8_t* bytes, size_t n, float* out) {
  switch (ty) {
    case T0R_F32:
      for (size_t i = 0; i < n; i++) memcpy(out + i, bytes + 4 * i, 4);
      return T0R_OK;
    case T0R_F16:
      for (size_t i = 0; i < n; i++) out[i] = t0r_f16_to_f32((uint16_t)(bytes[2 * i] | (bytes[2 * i + 1] << 8)));
      return T0R_OK;
    case T0R_Q8_0:
      if (n % QK) return T0R_ERR_SHAPE;
      t0r_dequantize_q8_0(bytes, n, out);
      return T0R_OK;
    case T0R_Q4_0:
      if (n % QK) return T0R_ERR_SHAPE;
      t0r_dequantize_q4_0(bytes, n, out);
      return T0R_OK;
  }
  return T0R_ERR_GGUF_TENSOR_TYPE;
}

/* gguf.rs:192-211 quantize_for */
int t0r_quantize_for(int ty, const float* x, size_t n, uint8_t* out) {
  switch (ty) {
    case T0R_F32:
      memcpy(out, x, n * 4);
      return T0R_OK;
    case T0R_F16:
      for (size_t i = 0; i < n; i++) {
        uint16_t h = t0r_f32_to_f16(x[i]);
        out[2 * i] = (uint8_t)(h & 0xff);
        out[2 * i + 1] = (uint8_t)(h >> 8);
      }
      return T0R_OK;
    case T0R_Q8_0:
      if (n % QK) return T0R_ERR_SHAPE;
      t0r_quantize_q8_0(x, n, out);
      return T0R_OK;
    case T0R_Q4_0:
      if (n % QK) return T0R_ERR_SHAPE;
      t0r_quantize_q4_0(x, n, out);
      return T0R_OK;
  }
  return T0R_ERR_GGUF_TENSOR_TYPE;
}

/* ------------------------------------------------------------------------- */
/* GGUF v3 container (gguf.rs:228-405)                                       */
/* ------------------------------------------------------------------------- */
enum { MV_U32 = 4, MV_F32 = 6, MV_BOOL = 7, MV_STRING = 8, MV_ARRAY = 9 };

typedef struct {
  char* key;
  int type;
  uint32_t u32;
  float f32;
  int boolean;
  char* str;
  float* arr;
  size_t arr_len;
} meta_t;

typedef struct {
  char* name;
  size_t shape[8];
  int rank;
  int ty;
  size_t n;
  float* data; /* dequantized f32 */
} tensor_t;

typedef struct {
  const float *norm, *w_qkv, *b_qkv, *w_o, *b_o, *q_norm, *k_norm, *mlp_norm, *w0, *b0, *w2, *b2;
  int is_group;
} layer_t;

typedef struct {
  const float *hw, *hb, *ow, *ob, *rw, *rb;
  size_t in_dim, hid, out_dim;
} rblock_t;

struct t0r_model {
  t0r_config cfg;
  char eps_mode[128];
  tensor_t* tensors;
  size_t n_tensors;
  rblock_t enc, dec;
  const float* type_emb;
  size_t n_types;
  layer_t* layers;
  const float* out_norm;
};

typedef struct {
  const uint8_t* p;
  size_t len, pos;
  int err;
} reader_t;

static int rd(reader_t* r, void* dst, size_t n) {
  if (r->err) return 0;
  if (n > r->len - r->pos) {
    r->err = T0R_ERR_GGUF_BOUNDS; /* UnexpectedEof in the reference */
    return 0;
  }
  memcpy(dst, r->p + r->pos, n);
  r->pos += n;
  return 1;
}
static uint32_t rd_u32(reader_t* r) {
  uint32_t v = 0;
  rd(r, &v, 4);
  return v;
}
static uint64_t rd_u64(reader_t* r) {
  uint64_t v = 0;
  rd(r, &v, 8);
  return v;
}

static int utf8_valid(const unsigned char* s, size_t n) {
  size_t i = 0;
  while (i < n) {
    unsigned c = s[i];
    size_t extra;
    uint32_t cp;
    if (c < 0x80) {
      i++;
      continue;
    } else if ((c & 0xe0) == 0xc0) {
      extra = 1;
      cp = c & 0x1f;
    } else if ((c & 0xf0) == 0xe0) {
      extra = 2;
      cp = c & 0x0f;
    } else if ((c & 0xf8) == 0xf0) {
      extra = 3;
      cp = c & 0x07;
    } else {
      return 0;
    }
    if (i + extra >= n) return 0;
    for (size_t k = 1; k <= extra; k++) {
      if ((s[i + k] & 0xc0) != 0x80) return 0;
      cp = (cp << 6) | (s[i + k] & 0x3f);
    }
    if ((extra == 1 && cp < 0x80) || (extra == 2 && cp < 0x800) || (extra == 3 && cp < 0x10000)) return 0;
    if (cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff)) return 0;
    i += extra + 1;
  }
  return 1;
}

/* gguf.rs:234-239 read_string */
static char* rd_string(reader_t* r) {
  uint64_t len = rd_u64(r);
  if (r->err) return NULL;
  if (len > r->len - r->pos) {
    r->err = T0R_ERR_GGUF_BOUNDS;
    return NULL;
  }
  char* s = (char*)malloc(len + 1);
  memcpy(s, r->p + r->pos, len);
  s[len] = 0;
  r->pos += len;
  if (!utf8_valid((const unsigned char*)s, len)) {
    r->err = T0R_ERR_METADATA;
    free(s);
    return NULL;
  }
  return s;
}

/* gguf.rs:271-292 read_meta_value */
static int rd_meta(reader_t* r, meta_t* m) {
  m->type = (int)rd_u32(r);
  if (r->err) return 0;
  switch (m->type) {
    case MV_U32: m->u32 = rd_u32(r); break;
    case MV_F32: rd(r, &m->f32, 4); break;
    case MV_BOOL: {
      uint8_t b = 0;
      rd(r, &b, 1);
      m->boolean = b != 0;
      break;
    }
    case MV_STRING: m->str = rd_string(r); break;
    case MV_ARRAY: {
      uint32_t et = rd_u32(r);
      uint64_t n = rd_u64(r);
      if (r->err) return 0;
      if (et != MV_F32) {
        r->err = T0R_ERR_GGUF_META_TYPE;
        return 0;
      }
      if (n > (r->len - r->pos) / 4) {
        r->err = T0R_ERR_GGUF_BOUNDS;
        return 0;
      }
      m->arr = (float*)malloc((n ? n : 1) * 4);
      m->arr_len = n;
      rd(r, m->arr, n * 4);
      break;
    }
    default: r->err = T0R_ERR_GGUF_META_TYPE; return 0;
  }
  return !r->err;
}

static void free_meta(meta_t* m, size_t n) {
  for (size_t i = 0; i < n; i++) {
    free(m[i].key);
    free(m[i].str);
    free(m[i].arr);
  }
  free(m);
}

/* HashMap insert semantics: a later key replaces an earlier one. */
static const meta_t* find_meta(const meta_t* m, size_t n, const char* key) {
  const meta_t* hit = NULL;
  for (size_t i = 0; i < n; i++)
    if (m[i].key && strcmp(m[i].key, key) == 0) hit = &m[i];
  return hit;
}

static const tensor_t* find_tensor(const t0r_model* mdl, const char* name) {
  const tensor_t* hit = NULL;
  for (size_t i = 0; i < mdl->n_tensors; i++)
    if (strcmp(mdl->tensors[i].name, name) == 0) hit = &mdl->tensors[i];
  return hit;
}

/* weights.rs:69-112 config_from_gguf_metadata */
static int config_from_meta(const meta_t* m, size_t n, t0r_config* cfg, char* eps_mode) {
  const char* req[6] = {"t0.embed_dim", "t0.num_layers", "t0.num_heads", "t0.mlp_hidden_dim", "t0.patch_size",
                        "t0.group_every_n"};
  uint32_t vals[6];
  for (int i = 0; i < 6; i++) {
    const meta_t* e = find_meta(m, n, req[i]);
    if (!e || e->type != MV_U32) return T0R_ERR_METADATA;
    vals[i] = e->u32;
  }
  const meta_t* ql = find_meta(m, n, "t0.quantile_levels");
  if (!ql || ql->type != MV_ARRAY) return T0R_ERR_METADATA;
  if (ql->arr_len == 0 || ql->arr_len > T0R_MAX_QUANTILES) return T0R_ERR_METADATA;
  memset(cfg, 0, sizeof(*cfg));
  cfg->embed_dim = vals[0];
  cfg->num_layers = vals[1];
  cfg->num_heads = vals[2];
  cfg->mlp_hidden_dim = vals[3];
  cfg->patch_size = vals[4];
  cfg->group_every_n = (int64_t)vals[5];
  const meta_t* e;
  e = find_meta(m, n, "t0.dropout");
  cfg->dropout = (e && e->type == MV_F32) ? e->f32 : 0.0f;
  cfg->n_quantiles = (uint32_t)ql->arr_len;
  memcpy(cfg->quantile_levels, ql->arr, ql->arr_len * 4);
  e = find_meta(m, n, "t0.scaler_use_arcsinh");
  cfg->scaler_use_arcsinh = (e && e->type == MV_BOOL) ? e->boolean : 1;
  e = find_meta(m, n, "t0.scaler_eps");
  cfg->scaler_eps = (e && e->type == MV_F32) ? e->f32 : 0.1f;
  e = find_meta(m, n, "t0.scaler_eps_mode");
  const char* mode = (e && e->type == MV_STRING) ? e->str : "variance_offset";
  snprintf(eps_mode, 128, "%s", mode);
  /* scaler.rs:28-34: anything but "std_clamp" is variance_offset */
  cfg->scaler_variance_offset = strcmp(mode, "std_clamp") != 0;
  return T0R_OK;
}

static int get_t(const t0r_model* m, const char* name, int rank, size_t d0, size_t d1, const float** out) {
  const tensor_t* t = find_tensor(m, name);
  if (!t) return T0R_ERR_MISSING_TENSOR;
  if (t->rank != rank) return T0R_ERR_SHAPE;
  if (rank >= 1 && d0 && t->shape[0] != d0) return T0R_ERR_SHAPE;
  if (rank >= 2 && d1 && t->shape[1] != d1) return T0R_ERR_SHAPE;
  *out = t->data;
  return T0R_OK;
}

/* model.rs:84-93 load_residual_block */
static int load_rblock(const t0r_model* m, const char* prefix, rblock_t* rb, size_t in_dim, size_t out_dim) {
  char nm[256];
  int rc;
  snprintf(nm, sizeof nm, "%s.mlp.hidden_layer.weight", prefix);
  const tensor_t* hw = find_tensor(m, nm);
  if (!hw) return T0R_ERR_MISSING_TENSOR;
  if (hw->rank != 2) return T0R_ERR_SHAPE;
  rb->hid = hw->shape[0];
  rb->in_dim = hw->shape[1];
  if (in_dim && rb->in_dim != in_dim) return T0R_ERR_SHAPE;
  rb->hw = hw->data;
  snprintf(nm, sizeof nm, "%s.mlp.hidden_layer.bias", prefix);
  if ((rc = get_t(m, nm, 1, rb->hid, 0, &rb->hb))) return rc;
  snprintf(nm, sizeof nm, "%s.mlp.output_layer.weight", prefix);
  const tensor_t* ow = find_tensor(m, nm);
  if (!ow) return T0R_ERR_MISSING_TENSOR;
  if (ow->rank != 2 || ow->shape[1] != rb->hid) return T0R_ERR_SHAPE;
  rb->out_dim = ow->shape[0];
  if (out_dim && rb->out_dim != out_dim) return T0R_ERR_SHAPE;
  rb->ow = ow->data;
  snprintf(nm, sizeof nm, "%s.mlp.output_layer.bias", prefix);
  if ((rc = get_t(m, nm, 1, rb->out_dim, 0, &rb->ob))) return rc;
  snprintf(nm, sizeof nm, "%s.residual_layer.weight", prefix);
  if ((rc = get_t(m, nm, 2, rb->out_dim, rb->in_dim, &rb->rw))) return rc;
  snprintf(nm, sizeof nm, "%s.residual_layer.bias", prefix);
  if ((rc = get_t(m, nm, 1, rb->out_dim, 0, &rb->rb))) return rc;
  return T0R_OK;
}

/* config.rs:45-56 layer_types */
static int layer_is_group(const t0r_config* c, size_t i) {
  if (c->group_every_n <= 0) return 0;
  size_t n = (size_t)c->group_every_n;
  size_t n_blocks = c->num_layers / n;
  if (i >= n_blocks * n) return -1; /* the reference's cycle().take() yields fewer layers */
  return (i % n) == n - 1;
}

void t0r_model_free(t0r_model* m) {
  if (!m) return;
  for (size_t i = 0; i < m->n_tensors; i++) {
    free(m->tensors[i].name);
    free(m->tensors[i].data);
  }
  free(m->tensors);
  free(m->layers);
  free(m);
}

/* gguf.rs:347-405 read_gguf + weights.rs:151-163 load_gguf_bytes + model.rs:108-147 T0Model::load */
int t0r_model_load_gguf(const uint8_t* bytes, size_t len, t0r_model** out) {
  *out = NULL;
  reader_t r = {bytes, len, 0, 0};
  char magic[4];
  if (!rd(&r, magic, 4)) return T0R_ERR_GGUF_MAGIC;
  if (memcmp(magic, "GGUF", 4) != 0) return T0R_ERR_GGUF_MAGIC;
  uint32_t version = rd_u32(&r);
  if (r.err) return r.err;
  if (version != 3) return T0R_ERR_GGUF_VERSION;
  uint64_t n_tensors = rd_u64(&r);
  uint64_t n_meta = rd_u64(&r);
  if (r.err) return r.err;
  if (n_meta > len || n_tensors > len) return T0R_ERR_GGUF_BOUNDS;
  meta_t* meta = (meta_t*)calloc(n_meta ? n_meta : 1, sizeof(meta_t));
  for (uint64_t i = 0; i < n_meta; i++) {
    meta[i].key = rd_string(&r);
    if (r.err) break;
    rd_meta(&r, &meta[i]);
    if (r.err) break;
  }
  if (r.err) {
    int e = r.err;
    free_meta(meta, n_meta);
    return e;
  }
  t0r_model* m = (t0r_model*)calloc(1, sizeof(t0r_model));
  m->tensors = (tensor_t*)calloc(n_tensors ? n_tensors : 1, sizeof(tensor_t));
  uint64_t* offsets = (uint64_t*)calloc(n_tensors ? n_tensors : 1, 8);
  int rc = T0R_OK;
  for (uint64_t i = 0; i < n_tensors && !rc; i++) {
    tensor_t* t = &m->tensors[i];
    t->name = rd_string(&r);
    uint32_t nd = rd_u32(&r);
    if (r.err) {
      rc = r.err;
      break;
    }
    if (nd > 8) {
      rc = T0R_ERR_SHAPE;
      break;
    }
    uint64_t ne[8];
    for (uint32_t k = 0; k < nd; k++) ne[k] = rd_u64(&r);
    t->rank = (int)nd;
    for (uint32_t k = 0; k < nd; k++) t->shape[k] = (size_t)ne[nd - 1 - k]; /* gguf.rs:381 reverse */
    uint32_t ty = rd_u32(&r);
    offsets[i] = rd_u64(&r);
    if (r.err) {
      rc = r.err;
      break;
    }
    if (ty != T0R_F32 && ty != T0R_F16 && ty != T0R_Q4_0 && ty != T0R_Q8_0) {
      rc = T0R_ERR_GGUF_TENSOR_TYPE;
      break;
    }
    t->ty = (int)ty;
    m->n_tensors = i + 1;
  }
  if (!rc) {
    /* everything after the tensor infos is the blob (gguf.rs:387-389) */
    const uint8_t* blob = bytes + r.pos;
    size_t blob_len = len - r.pos;
    for (uint64_t i = 0; i < n_tensors && !rc; i++) {
      tensor_t* t = &m->tensors[i];
      size_t n = 1;
      for (int k = 0; k < t->rank; k++) n *= t->shape[k];
      size_t nbytes = t0r_row_bytes(t->ty, n);
      if (nbytes == 0 && n != 0) {
        rc = T0R_ERR_SHAPE;
        break;
      }
      if (offsets[i] > blob_len || nbytes > blob_len - offsets[i]) {
        rc = T0R_ERR_GGUF_BOUNDS;
        break;
      }
      t->n = n;
      t->data = (float*)malloc((n ? n : 1) * sizeof(float));
      if (!t->data) {
        rc = T0R_ERR_OOM;
        break;
      }
      t0r_dequantize_for(t->ty, blob + offsets[i], n, t->data);
    }
  }
  free(offsets);
  if (!rc) rc = config_from_meta(meta, n_meta, &m->cfg, m->eps_mode);
  free_meta(meta, n_meta);
  if (rc) {
    t0r_model_free(m);
    return rc;
  }

  /* model.rs:108-147 T0Model::load */
  t0r_config* c = &m->cfg;
  if (c->num_heads == 0 || c->embed_dim % c->num_heads || (c->embed_dim / c->num_heads) % 2 || c->patch_size == 0) {
    t0r_model_free(m);
    return T0R_ERR_METADATA;
  }
  size_t E = c->embed_dim, H = c->mlp_hidden_dim;
  rc = load_rblock(m, "patch_encoder.projection", &m->enc, 3 * (size_t)c->patch_size, E);
  if (!rc) {
    const tensor_t* te = find_tensor(m, "patch_encoder.type_embeddings.weight");
    if (!te) rc = T0R_ERR_MISSING_TENSOR;
    else if (te->rank != 2 || te->shape[1] != E) rc = T0R_ERR_SHAPE;
    else {
      m->type_emb = te->data;
      m->n_types = te->shape[0];
    }
  }
  size_t n_layers = c->num_layers;
  if (c->group_every_n > 0) n_layers = (c->num_layers / (size_t)c->group_every_n) * (size_t)c->group_every_n;
  m->layers = (layer_t*)calloc(n_layers ? n_layers : 1, sizeof(layer_t));
  for (size_t i = 0; i < n_layers && !rc; i++) {
    layer_t* L = &m->layers[i];
    char nm[256];
    L->is_group = layer_is_group(c, i) == 1;
    size_t hd = E / c->num_heads;
#define GT(rank, d0, d1, dst, fmt)                   \
  snprintf(nm, sizeof nm, fmt, i);                   \
  if (!rc) rc = get_t(m, nm, rank, d0, d1, &L->dst);
    GT(1, E, 0, norm, "transformer.layers.%zu.attention_block.norm.scale");
    GT(2, 3 * E, E, w_qkv, "transformer.layers.%zu.attention_block.attention.wQKV.weight");
    GT(1, 3 * E, 0, b_qkv, "transformer.layers.%zu.attention_block.attention.wQKV.bias");
    GT(2, E, E, w_o, "transformer.layers.%zu.attention_block.attention.wO.weight");
    GT(1, E, 0, b_o, "transformer.layers.%zu.attention_block.attention.wO.bias");
    GT(1, hd, 0, q_norm, "transformer.layers.%zu.attention_block.attention.q_norm.scale");
    GT(1, hd, 0, k_norm, "transformer.layers.%zu.attention_block.attention.k_norm.scale");
    GT(1, E, 0, mlp_norm, "transformer.layers.%zu.norm.scale");
    GT(2, 2 * H, E, w0, "transformer.layers.%zu.mlp.0.weight");
    GT(1, 2 * H, 0, b0, "transformer.layers.%zu.mlp.0.bias");
    GT(2, E, H, w2, "transformer.layers.%zu.mlp.2.weight");
    GT(1, E, 0, b2, "transformer.layers.%zu.mlp.2.bias");
#undef GT
  }
  c->num_layers = (uint32_t)n_layers;
  if (!rc) rc = get_t(m, "transformer.out_norm.scale", 1, E, 0, &m->out_norm);
  if (!rc) rc = load_rblock(m, "decoder", &m->dec, E, (size_t)c->patch_size * c->n_quantiles);
  if (rc) {
    t0r_model_free(m);
    return rc;
  }
  *out = m;
  return T0R_OK;
}

int t0r_model_config(const t0r_model* m, t0r_config* out) {
  if (!m || !out) return T0R_ERR_INVALID_ARG;
  *out = m->cfg;
  return T0R_OK;
}

size_t t0r_model_tensor_count(const t0r_model* m) { return m ? m->n_tensors : 0; }

size_t t0r_model_tensor(const t0r_model* m, const char* name, float* out, size_t cap, size_t shape[4], int* rank) {
  const tensor_t* t = find_tensor(m, name);
  if (!t) return 0;
  if (out) memcpy(out, t->data, (t->n < cap ? t->n : cap) * sizeof(float));
  if (shape)
    for (int k = 0; k < 4; k++) shape[k] = k < t->rank ? t->shape[k] : 0;
  if (rank) *rank = t->rank;
  return t->n;
}

/* ---- GGUF writer (gguf.rs:299-345) + export policy (weights.rs:32-37, 187-227) ---- */
typedef struct {
  uint8_t* p;
  size_t cap, pos;
} writer_t;
static void wr(writer_t* w, const void* src, size_t n) {
  if (w->p && w->pos + n <= w->cap) memcpy(w->p + w->pos, src, n);
  w->pos += n;
}
static void wr_u32(writer_t* w, uint32_t v) { wr(w, &v, 4); }
static void wr_u64(writer_t* w, uint64_t v) { wr(w, &v, 8); }
static void wr_str(writer_t* w, const char* s) {
  wr_u64(w, strlen(s));
  wr(w, s, strlen(s));
}

/* weights.rs:32-37 is_quantizable */
static int is_quantizable(const char* name) {
  return strstr(name, ".attention.wQKV.weight") || strstr(name, ".attention.wO.weight") ||
         strstr(name, ".mlp.0.weight") || strstr(name, ".mlp.2.weight");
}

static int cmp_tensor_name(const void* a, const void* b) {
  const tensor_t* x = *(const tensor_t* const*)a;
  const tensor_t* y = *(const tensor_t* const*)b;
  return strcmp(x->name, y->name);
}

size_t t0r_export_gguf(const t0r_model* m, int quant, uint8_t* out, size_t cap) {
  writer_t w = {out, cap, 0};
  size_t n = m->n_tensors;
  /* de-duplicate by name (HashMap semantics: the last definition wins) */
  const tensor_t** sorted = (const tensor_t**)malloc((n ? n : 1) * sizeof(*sorted));
  size_t ns = 0;
  for (size_t i = 0; i < n; i++)
    if (find_tensor(m, m->tensors[i].name) == &m->tensors[i]) sorted[ns++] = &m->tensors[i];
  qsort(sorted, ns, sizeof(*sorted), cmp_tensor_name);
  int* types = (int*)malloc((ns ? ns : 1) * sizeof(int));
  size_t* sizes = (size_t*)malloc((ns ? ns : 1) * sizeof(size_t));
  for (size_t i = 0; i < ns; i++) {
    const tensor_t* t = sorted[i];
    int ty;
    if (quant == T0R_F32) ty = T0R_F32;
    else ty = (t->rank == 2 && is_quantizable(t->name)) ? quant : T0R_F16; /* weights.rs:195-199 */
    types[i] = ty;
    sizes[i] = t0r_row_bytes(ty, t->n);
  }
  wr(&w, "GGUF", 4);
  wr_u32(&w, 3);
  wr_u64(&w, ns);
  wr_u64(&w, 11);
  /* weights.rs:208-220: key order and value types */
  const t0r_config* c = &m->cfg;
  wr_str(&w, "t0.embed_dim"); wr_u32(&w, MV_U32); wr_u32(&w, c->embed_dim);
  wr_str(&w, "t0.num_layers"); wr_u32(&w, MV_U32); wr_u32(&w, c->num_layers);
  wr_str(&w, "t0.num_heads"); wr_u32(&w, MV_U32); wr_u32(&w, c->num_heads);
  wr_str(&w, "t0.mlp_hidden_dim"); wr_u32(&w, MV_U32); wr_u32(&w, c->mlp_hidden_dim);
  wr_str(&w, "t0.patch_size"); wr_u32(&w, MV_U32); wr_u32(&w, c->patch_size);
  wr_str(&w, "t0.group_every_n"); wr_u32(&w, MV_U32); wr_u32(&w, (uint32_t)c->group_every_n);
  wr_str(&w, "t0.dropout"); wr_u32(&w, MV_F32); wr(&w, &c->dropout, 4);
  wr_str(&w, "t0.quantile_levels"); wr_u32(&w, MV_ARRAY); wr_u32(&w, MV_F32); wr_u64(&w, c->n_quantiles);
  wr(&w, c->quantile_levels, 4 * (size_t)c->n_quantiles);
  wr_str(&w, "t0.scaler_use_arcsinh"); wr_u32(&w, MV_BOOL);
  uint8_t b = c->scaler_use_arcsinh ? 1 : 0;
  wr(&w, &b, 1);
  wr_str(&w, "t0.scaler_eps"); wr_u32(&w, MV_F32); wr(&w, &c->scaler_eps, 4);
  wr_str(&w, "t0.scaler_eps_mode"); wr_u32(&w, MV_STRING); wr_str(&w, m->eps_mode);
  /* offsets relative to the blob, 32-aligned (gguf.rs:310-320) */
  uint64_t cursor = 0;
  uint64_t* offs = (uint64_t*)malloc((ns ? ns : 1) * 8);
  for (size_t i = 0; i < ns; i++) {
    offs[i] = cursor;
    cursor += sizes[i];
    if (cursor % 32) cursor += 32 - cursor % 32;
  }
  for (size_t i = 0; i < ns; i++) {
    const tensor_t* t = sorted[i];
    wr_str(&w, t->name);
    wr_u32(&w, (uint32_t)t->rank);
    for (int k = t->rank - 1; k >= 0; k--) wr_u64(&w, t->shape[k]);
    wr_u32(&w, (uint32_t)types[i]);
    wr_u64(&w, offs[i]);
  }
  /* blob right after the infos, unaligned in the file (gguf.rs:333-344) */
  uint64_t pos = 0;
  for (size_t i = 0; i < ns; i++) {
    uint8_t zero = 0;
    for (uint64_t k = pos; k < offs[i]; k++) wr(&w, &zero, 1);
    uint8_t* buf = (uint8_t*)malloc(sizes[i] ? sizes[i] : 1);
    t0r_quantize_for(types[i], sorted[i]->data, sorted[i]->n, buf);
    wr(&w, buf, sizes[i]);
    free(buf);
    pos = offs[i] + sizes[i];
  }
  free(offs);
  free(types);
  free(sizes);
  free(sorted);
  return w.pos;
}

static int g_threads = 0;
void t0r_set_threads(int n) { g_threads = n; }
static int nthreads(void) {
#ifdef _OPENMP
  return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------------- */
/* ops (ops.rs)                                                              */
/* ------------------------------------------------------------------------- */

/* f32 dot with a fixed 8-way split; independent of thread count and ISA. */
static float dot8(const float* a, const float* b, size_t k) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t i = 0;
  for (; i + 8 <= k; i += 8)
    for (int l = 0; l < 8; l++) acc[l] += a[i + l] * b[i + l];
  for (; i < k; i++) acc[i & 7] += a[i] * b[i];
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

/* ops.rs:40-42 linear: y = x @ w^T + b (w is [n, k]); optional relu (ops.rs:33) */
void t0r_linear(const float* x, const float* w, const float* b, float* y, size_t m, size_t k, size_t n, int relu) {
  const size_t NB = 32;
#pragma omp parallel for schedule(dynamic, 1) collapse(2) num_threads(nthreads())
  for (size_t mb = 0; mb < (m + 15) / 16; mb++)
    for (size_t nb = 0; nb < (n + NB - 1) / NB; nb++) {
      size_t m_end = (mb + 1) * 16 < m ? (mb + 1) * 16 : m;
      size_t n_end = (nb + 1) * NB < n ? (nb + 1) * NB : n;
      for (size_t i = mb * 16; i < m_end; i++)
        for (size_t j = nb * NB; j < n_end; j++) {
          float v = dot8(x + i * k, w + j * k, k);
          if (b) v = v + b[j];
          if (relu) v = v > 0.0f ? v : 0.0f;
          y[i * n + j] = v;
        }
    }
}

/* ops.rs:12-17 rmsnorm: x / sqrt(mean(x^2) + eps) * scale */
void t0r_rmsnorm(const float* x, const float* scale, float* y, size_t rows, size_t dim, float eps) {
#pragma omp parallel for schedule(static) num_threads(nthreads()) if (rows * dim > 65536)
  for (size_t r = 0; r < rows; r++) {
    const float* xr = x + r * dim;
    float ss = 0.0f;
    for (size_t d = 0; d < dim; d++) ss += xr[d] * xr[d];
    float ms = ss / (float)dim;
    float denom = sqrtf(ms + eps);
    for (size_t d = 0; d < dim; d++) y[r * dim + d] = (xr[d] / denom) * scale[d];
  }
}

/* ops.rs:77-116 RopeTables::new (f64 math, f32 tables; theta 10000, xpos base 512) */
void t0r_rope_tables(size_t seq_len, size_t head_dim, float* cos_t, float* sin_t, float* scale_t) {
  size_t half = head_dim / 2;
  double theta = 10000.0, scale_base = 512.0;
  double max_pos = (double)(seq_len - 1);
  double max_half = floor(max_pos / 2.0);
  for (size_t p = 0; p < seq_len; p++) {
    double power = ((double)p - max_half) / scale_base;
    for (size_t j = 0; j < half; j++) {
      double inv_freq = 1.0 / pow(theta, (double)(2 * j) / (double)head_dim);
      double angle = (double)p * inv_freq;
      double base = (2.0 * (double)j + 0.4 * (double)head_dim) / (1.4 * (double)head_dim);
      float s = (float)pow(base, power);
      for (int k = 0; k < 2; k++) {
        size_t idx = p * head_dim + 2 * j + (size_t)k;
        cos_t[idx] = (float)cos(angle);
        sin_t[idx] = (float)sin(angle);
      }
      scale_t[p * head_dim + j] = s;
      scale_t[p * head_dim + half + j] = s;
    }
  }
}

/* silu as silu_mul.wgsl:21 (g / (1 + exp(-g))), softplus as quantile_head.wgsl:19 */
static float silu(float g) { return g / (1.0f + expf(-g)); }
static float softplus(float x) { return logf(1.0f + expf(x)); }

/* ops.rs:195-210 quantile_head */
void t0r_quantile_head(const float* x, float* y, size_t rows, size_t n_q) {
  for (size_t r = 0; r < rows; r++) {
    const float* xr = x + r * n_q;
    float running = xr[0];
    y[r * n_q] = running;
    for (size_t i = 1; i < n_q; i++) {
      running = running + softplus(xr[i]);
      y[r * n_q + i] = running;
    }
  }
}

/* ------------------------------------------------------------------------- */
/* quantile.rs                                                               */
/* ------------------------------------------------------------------------- */
typedef struct {
  float key;
  size_t idx;
} kidx_t;
/* stable order: Rust's sort_by is stable, so ties keep their input order */
static int cmp_kidx(const void* a, const void* b) {
  const kidx_t* x = (const kidx_t*)a;
  const kidx_t* y = (const kidx_t*)b;
  if (x->key < y->key) return -1;
  if (x->key > y->key) return 1;
  return x->idx < y->idx ? -1 : (x->idx > y->idx ? 1 : 0);
}

/* quantile.rs:16-41 interpolate_quantiles */
void t0r_interpolate_quantiles(const float* query, size_t nq, const float* orig_levels, const float* orig_values,
                               size_t nl, float* out) {
  if (nl == 0) return; /* the reference unwraps first()/last() and panics */
  kidx_t* ki = (kidx_t*)malloc(nl * sizeof(kidx_t));
  for (size_t i = 0; i < nl; i++) {
    ki[i].key = orig_levels[i];
    ki[i].idx = i;
  }
  qsort(ki, nl, sizeof(kidx_t), cmp_kidx);
  float* levels = (float*)malloc((nl + 2) * sizeof(float));
  float* values = (float*)malloc((nl + 2) * sizeof(float));
  size_t n = 0;
  if (orig_levels[ki[0].idx] > 0.0f) {
    levels[n] = 0.0f;
    values[n] = orig_values[ki[0].idx];
    n++;
  }
  for (size_t i = 0; i < nl; i++) {
    levels[n] = orig_levels[ki[i].idx];
    values[n] = orig_values[ki[i].idx];
    n++;
  }
  if (levels[n - 1] < 1.0f) {
    levels[n] = 1.0f;
    values[n] = values[n - 1];
    n++;
  }
  for (size_t qi = 0; qi < nq; qi++) {
    float q = query[qi];
    size_t upper = 0;
    while (upper < n && levels[upper] <= q) upper++; /* partition_point(l <= q) */
    if (upper > n - 1) upper = n - 1;
    size_t lower = upper > 0 ? upper - 1 : 0;
    float ll = levels[lower], ul = levels[upper], lv = values[lower], uv = values[upper];
    float diff = ul - ll;
    float w = diff == 0.0f ? 0.0f : (q - ll) / diff;
    out[qi] = lv + w * (uv - lv);
  }
  free(ki);
  free(levels);
  free(values);
}

/* quantile.rs:45-59 weighted_quantile */
void t0r_weighted_quantile(const float* query, size_t nq, const float* weights, const float* samples, size_t ns,
                           float* out) {
  float sum = 0.0f;
  for (size_t i = 0; i < ns; i++) sum += weights[i];
  kidx_t* ki = (kidx_t*)malloc(ns * sizeof(kidx_t));
  for (size_t i = 0; i < ns; i++) {
    ki[i].key = samples[i];
    ki[i].idx = i;
  }
  qsort(ki, ns, sizeof(kidx_t), cmp_kidx);
  float* sorted = (float*)malloc(ns * sizeof(float));
  float* cumul = (float*)malloc(ns * sizeof(float));
  float cum = 0.0f;
  for (size_t i = 0; i < ns; i++) {
    sorted[i] = samples[ki[i].idx];
    cum += weights[ki[i].idx] / sum;
    float c = cum;
    if (c < 0.0f) c = 0.0f;
    if (c > 1.0f) c = 1.0f;
    cumul[i] = c;
  }
  t0r_interpolate_quantiles(query, nq, cumul, sorted, ns, out);
  free(ki);
  free(sorted);
  free(cumul);
}

/* quantile.rs:64-76 prob_mass */
void t0r_prob_mass(const float* levels, size_t n, float* out) {
  float* bnd = (float*)malloc((n + 2) * sizeof(float));
  bnd[0] = 0.0f;
  for (size_t i = 0; i < n; i++) bnd[i + 1] = levels[i];
  bnd[n + 1] = 1.0f;
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) {
    out[i] = (bnd[i + 2] - bnd[i]) / 2.0f;
    sum += out[i];
  }
  for (size_t i = 0; i < n; i++) out[i] /= sum;
  free(bnd);
}

/* ------------------------------------------------------------------------- */
/* host prep: data.rs, scaler.rs, mask.rs                                     */
/* ------------------------------------------------------------------------- */
enum { MT_VALID = 0, MT_PAD = 1, MT_MISSING = 2, MT_CENSORED = 3, MT_WITHHELD = 4 };
enum { VT_TARGET = 0, VT_HISTORICAL = 1, VT_FUTURE = 2 };

typedef struct {
  size_t v, t;
  float* variates;
  int8_t* mask;
  int64_t* group_ids;
  int64_t* variate_type;
} series_t;

static void series_alloc(series_t* s, size_t v, size_t t) {
  s->v = v;
  s->t = t;
  size_t n = (v * t != 0) ? v * t : 1;
  s->variates = (float*)calloc(n, sizeof(float));
  s->mask = (int8_t*)calloc(n, 1);
  s->group_ids = (int64_t*)calloc(n, 8);
  s->variate_type = (int64_t*)calloc(n, 8);
}
static void series_free(series_t* s) {
  free(s->variates);
  free(s->mask);
  free(s->group_ids);
  free(s->variate_type);
}

/* data.rs:52-86 TimeSeries::from_context */
static void from_context(const float* ctx, size_t v, size_t t_ctx, size_t horizon, series_t* s) {
  size_t t = t_ctx + horizon;
  series_alloc(s, v, t);
  for (size_t row = 0; row < v; row++) {
    for (size_t col = 0; col < t_ctx; col++) {
      size_t idx = row * t + col;
      float x = ctx[row * t_ctx + col];
      if (isnan(x)) {
        s->variates[idx] = 0.0f;
        s->mask[idx] = MT_MISSING;
      } else {
        s->variates[idx] = x;
        s->mask[idx] = MT_VALID;
      }
    }
    for (size_t col = t_ctx; col < t; col++) {
      s->variates[row * t + col] = 0.0f;
      s->mask[row * t + col] = MT_WITHHELD;
    }
    for (size_t col = 0; col < t; col++) {
      s->group_ids[row * t + col] = 0;
      s->variate_type[row * t + col] = VT_TARGET;
    }
  }
}

/* data.rs:110-155 TimeSeries::pad */
static void series_pad(const series_t* in, size_t patch, size_t context_end, series_t* out) {
  size_t horizon = in->t - context_end;
  size_t pad_left = (patch - context_end % patch) % patch;
  size_t pad_right = ((horizon + patch - 1) / patch) * patch - horizon;
  size_t new_t = pad_left + in->t + pad_right;
  size_t v = in->v;
  series_alloc(out, v, new_t);
  for (size_t i = 0; i < v * new_t; i++) {
    out->mask[i] = MT_PAD;
    out->group_ids[i] = -1;
    out->variate_type[i] = -1;
  }
  for (size_t row = 0; row < v; row++) {
    int64_t row_group = in->group_ids[row * in->t + in->t - 1];
    int64_t row_type = in->variate_type[row * in->t + in->t - 1];
    for (size_t col = 0; col < in->t; col++) {
      size_t src = row * in->t + col, dst = row * new_t + pad_left + col;
      out->variates[dst] = in->variates[src];
      out->mask[dst] = in->mask[src];
      out->group_ids[dst] = in->group_ids[src];
      out->variate_type[dst] = in->variate_type[src];
    }
    int is_target = row_type == VT_TARGET;
    for (size_t col = 0; col < pad_right; col++) {
      size_t dst = row * new_t + pad_left + in->t + col;
      out->group_ids[dst] = row_group;
      out->variate_type[dst] = row_type;
      out->mask[dst] = is_target ? MT_WITHHELD : MT_PAD;
    }
  }
}

/* Rust 1.99 std f32::asinh (library/std/src/f32.rs): ln_1p(ax + ax/(hypot(1, 1/ax) + 1/ax)) with sign */
static float rust_asinhf(float x) {
  float ax = fabsf(x);
  float ix = 1.0f / ax;
  return copysignf(log1pf(ax + (ax / (hypotf(1.0f, ix) + ix))), x);
}

/* scaler.rs:91-118 causal_row_stats (Welford, emit after update) */
static void causal_row_stats(const float* x, const int8_t* mask, size_t t, float eps, int variance_offset, float* loc,
                             float* scale) {
  float count = 0.0f, mean = 0.0f, m2 = 0.0f;
  for (size_t col = 0; col < t; col++) {
    if (mask[col] == MT_VALID) {
      count += 1.0f;
      float delta = x[col] - mean;
      mean += delta / count;
      float delta2 = x[col] - mean;
      m2 += delta * delta2;
    }
    loc[col] = mean;
    float variance = count > 1.0f ? fmaxf(m2 / (count - 1.0f), 0.0f) : 0.0f;
    scale[col] = variance_offset ? sqrtf(variance + eps) : fmaxf(sqrtf(variance), eps);
  }
}

/* scaler.rs:44-86 scale_input */
int t0r_scale_input(const float* variates, const int8_t* mask, const int64_t* group_ids, const int64_t* variate_type,
                    size_t v, size_t t, int use_arcsinh, float eps, int variance_offset, float* scaled, float* loc,
                    float* scale) {
  for (size_t i = 0; i < v * t; i++)
    if (variate_type[i] == VT_FUTURE) return T0R_ERR_FUTURE_ROWS;
  for (size_t row = 0; row < v; row++) {
    size_t base = row * t;
    causal_row_stats(variates + base, mask + base, t, eps, variance_offset, loc + base, scale + base);
    for (size_t col = 0; col < t; col++)
      if (group_ids[base + col] < 0) {
        loc[base + col] = 0.0f;
        scale[base + col] = 1.0f;
      }
  }
  for (size_t i = 0; i < v * t; i++) {
    float x = (variates[i] - loc[i]) / scale[i];
    scaled[i] = use_arcsinh ? rust_asinhf(x) : x;
  }
  return T0R_OK;
}

/* mask.rs:12-28 reduce_patch_metadata */
static void reduce_patch_metadata(const int64_t* meta, const int8_t* mask, size_t v, size_t t, size_t patch,
                                  int64_t* out) {
  size_t p = t / patch;
  for (size_t row = 0; row < v; row++)
    for (size_t pi = 0; pi < p; pi++) {
      size_t base = row * t + pi * patch;
      out[row * p + pi] = -1;
      for (size_t k = 0; k < patch; k++)
        if (mask[base + k] != MT_PAD) {
          out[row * p + pi] = meta[base + k];
          break;
        }
    }
}

/* mask.rs:32-43 patch_attendable */
static void patch_attendable(const int8_t* mask, size_t v, size_t t, size_t patch, uint8_t* out) {
  size_t p = t / patch;
  for (size_t row = 0; row < v; row++)
    for (size_t pi = 0; pi < p; pi++) {
      size_t base = row * t + pi * patch;
      uint8_t any = 0;
      for (size_t k = 0; k < patch; k++)
        if (mask[base + k] != MT_PAD) any = 1;
      out[row * p + pi] = any;
    }
}

#define BLOCK_F (-1.0e9f) /* mask.rs:8 */

/* mask.rs:49-65 build_time_mask, [v, p, p] */
void t0r_build_time_mask(const int64_t* pg, const int64_t* pvt, const uint8_t* att, size_t v, size_t p, float* out) {
  for (size_t row = 0; row < v; row++) {
    int is_future = pvt[row * p] == VT_FUTURE;
    for (size_t i = 0; i < p; i++)
      for (size_t j = 0; j < p; j++) {
        int64_t gi = pg[row * p + i], gj = pg[row * p + j];
        int same = gi >= 0 && gi == gj;
        int causal = is_future || j <= i;
        int attend = same && causal && att[row * p + j];
        out[row * p * p + i * p + j] = attend ? 0.0f : BLOCK_F;
      }
  }
}

/* mask.rs:69-82 build_group_mask, [p, v, v] */
void t0r_build_group_mask(const int64_t* pg, size_t v, size_t p, float* out) {
  for (size_t pi = 0; pi < p; pi++)
    for (size_t i = 0; i < v; i++)
      for (size_t j = 0; j < v; j++) {
        int64_t gi = pg[i * p + pi], gj = pg[j * p + pi];
        out[pi * v * v + i * v + j] = (gi >= 0 && gi == gj) ? 0.0f : BLOCK_F;
      }
}

/* ------------------------------------------------------------------------- */
/* forward (model.rs:177-300)                                                */
/* ------------------------------------------------------------------------- */

/* ops.rs:24-37 residual_block: mlp(x) + residual_layer(x) */
static void residual_block(const rblock_t* rb, const float* x, size_t rows, float* out) {
  float* hidden = (float*)malloc(rows * rb->hid * sizeof(float));
  float* res = (float*)malloc(rows * rb->out_dim * sizeof(float));
  t0r_linear(x, rb->hw, rb->hb, hidden, rows, rb->in_dim, rb->hid, 1);
  t0r_linear(hidden, rb->ow, rb->ob, out, rows, rb->hid, rb->out_dim, 0);
  t0r_linear(x, rb->rw, rb->rb, res, rows, rb->in_dim, rb->out_dim, 0);
  for (size_t i = 0; i < rows * rb->out_dim; i++) out[i] = out[i] + res[i];
  free(hidden);
  free(res);
}

/* ops.rs:153-190 mhsa.  x: rows ordered (outer, seq); mask: [mask_outer, seq, seq]
 * (mask_outer is `outer`).  rope tables [seq, hd] or NULL. out: [outer*seq, E]. */
static void mhsa(const t0r_model* m, const layer_t* L, const float* x, size_t outer, size_t seq, const float* mask,
                 const float* cos_t, const float* sin_t, const float* sc_t, float* out) {
  size_t E = m->cfg.embed_dim, H = m->cfg.num_heads, hd = E / H, rows = outer * seq;
  float* qkv = (float*)malloc(rows * 3 * E * sizeof(float));
  t0r_linear(x, L->w_qkv, L->b_qkv, qkv, rows, E, 3 * E, 0);
  float* att = (float*)malloc(rows * E * sizeof(float));
  const float scale = 1.0f / sqrtf((float)hd);
#pragma omp parallel num_threads(nthreads()) if (rows * H * seq > 20000)
  {
    float* q = (float*)malloc(seq * hd * sizeof(float));
    float* k = (float*)malloc(seq * hd * sizeof(float));
    float* sc = (float*)malloc(seq * sizeof(float));
#pragma omp for schedule(dynamic, 1) collapse(2)
    for (size_t o = 0; o < outer; o++)
      for (size_t h = 0; h < H; h++) {
        /* qk rmsnorm per head (ops.rs:175-177), then rope (ops.rs:178-181) */
        for (size_t s = 0; s < seq; s++) {
          const float* row = qkv + (o * seq + s) * 3 * E;
          for (int which = 0; which < 2; which++) {
            const float* src = row + (size_t)which * E + h * hd;
            const float* nscale = which ? L->k_norm : L->q_norm;
            float* dst = (which ? k : q) + s * hd;
            float ss = 0.0f;
            for (size_t d = 0; d < hd; d++) ss += src[d] * src[d];
            float denom = sqrtf(ss / (float)hd + 1e-8f);
            float tmp[512];
            for (size_t d = 0; d < hd; d++) tmp[d] = (src[d] / denom) * nscale[d];
            if (cos_t) {
              /* ops.rs:132-142: x*cos*scale + rotate_half(x)*sin*scale; k uses scale.recip() */
              for (size_t d = 0; d < hd; d++) {
                float c = cos_t[s * hd + d], sn = sin_t[s * hd + d], xs = sc_t[s * hd + d];
                float sv = which ? 1.0f / xs : xs;
                float rot = (d % 2 == 0) ? -tmp[d + 1] : tmp[d - 1];
                dst[d] = ((tmp[d] * c) * sv) + ((rot * sn) * sv);
              }
            } else {
              for (size_t d = 0; d < hd; d++) dst[d] = tmp[d];
            }
          }
        }
        for (size_t i = 0; i < seq; i++) {
          float mx = -INFINITY;
          for (size_t j = 0; j < seq; j++) {
            float s = dot8(q + i * hd, k + j * hd, hd) * scale;
            s = s + mask[o * seq * seq + i * seq + j];
            sc[j] = s;
            mx = fmaxf(mx, s);
          }
          float sum = 0.0f;
          for (size_t j = 0; j < seq; j++) {
            sc[j] = expf(sc[j] - mx);
            sum += sc[j];
          }
          for (size_t j = 0; j < seq; j++) sc[j] = sc[j] / sum;
          float* dst = att + (o * seq + i) * E + h * hd;
          for (size_t d = 0; d < hd; d++) dst[d] = 0.0f;
          for (size_t j = 0; j < seq; j++) {
            const float* vr = qkv + (o * seq + j) * 3 * E + 2 * E + h * hd;
            for (size_t d = 0; d < hd; d++) dst[d] += sc[j] * vr[d];
          }
        }
      }
    free(q);
    free(k);
    free(sc);
  }
  t0r_linear(att, L->w_o, L->b_o, out, rows, E, E, 0);
  free(att);
  free(qkv);
}

/* ops.rs:49-62 swiglu_ffn */
static void swiglu(const t0r_model* m, const layer_t* L, const float* x, size_t rows, float* out) {
  size_t E = m->cfg.embed_dim, H = m->cfg.mlp_hidden_dim;
  float* hid = (float*)malloc(rows * 2 * H * sizeof(float));
  float* g = (float*)malloc(rows * H * sizeof(float));
  t0r_linear(x, L->w0, L->b0, hid, rows, E, 2 * H, 0);
  for (size_t r = 0; r < rows; r++)
    for (size_t j = 0; j < H; j++) g[r * H + j] = silu(hid[r * 2 * H + j]) * hid[r * 2 * H + H + j];
  t0r_linear(g, L->w2, L->b2, out, rows, H, E, 0);
  free(hid);
  free(g);
}

static int forward_series(const t0r_model* m, const series_t* s, float* out, float* tr_pe, float* tr_l0) {
  const t0r_config* c = &m->cfg;
  size_t v = s->v, ps = c->patch_size, E = c->embed_dim, hd = E / c->num_heads;
  if (s->t % ps) return T0R_ERR_SHAPE;
  size_t p = s->t / ps, rows = v * p;
  if (rows == 0) return T0R_OK;
  /* patch encoder input, model.rs:185-197 */
  float* concat = (float*)malloc(rows * ps * 3 * sizeof(float));
  for (size_t row = 0; row < v; row++)
    for (size_t pi = 0; pi < p; pi++)
      for (size_t k = 0; k < ps; k++) {
        size_t src = row * s->t + pi * ps + k, base = (row * p + pi) * ps * 3;
        concat[base + k] = s->variates[src];
        concat[base + ps + k] = (float)k / (float)ps;
        concat[base + 2 * ps + k] = s->mask[src] == MT_VALID ? 1.0f : 0.0f;
      }
  float* x = (float*)malloc(rows * E * sizeof(float));
  residual_block(&m->enc, concat, rows, x);
  free(concat);
  int64_t* pvt = (int64_t*)malloc(rows * 8);
  int64_t* pg = (int64_t*)malloc(rows * 8);
  uint8_t* att = (uint8_t*)malloc(rows);
  reduce_patch_metadata(s->variate_type, s->mask, v, s->t, ps, pvt);
  reduce_patch_metadata(s->group_ids, s->mask, v, s->t, ps, pg);
  patch_attendable(s->mask, v, s->t, ps, att);
  /* model.rs:205-207 type embedding, index max(type, 0) */
  for (size_t r = 0; r < rows; r++) {
    int64_t ti = pvt[r] > 0 ? pvt[r] : 0;
    if ((size_t)ti >= m->n_types) {
      free(x);
      free(pvt);
      free(pg);
      free(att);
      return T0R_ERR_INVALID_ARG;
    }
    for (size_t e = 0; e < E; e++) x[r * E + e] = x[r * E + e] + m->type_emb[(size_t)ti * E + e];
  }
  if (tr_pe) memcpy(tr_pe, x, rows * E * sizeof(float));
  float* tmask = (float*)malloc(v * p * p * sizeof(float));
  float* gmask = (float*)malloc(p * v * v * sizeof(float));
  t0r_build_time_mask(pg, pvt, att, v, p, tmask);
  t0r_build_group_mask(pg, v, p, gmask);
  float* ct = (float*)malloc(p * hd * sizeof(float));
  float* st = (float*)malloc(p * hd * sizeof(float));
  float* xt = (float*)malloc(p * hd * sizeof(float));
  t0r_rope_tables(p, hd, ct, st, xt);

  float* normed = (float*)malloc(rows * E * sizeof(float));
  float* tmp = (float*)malloc(rows * E * sizeof(float));
  float* tmp2 = (float*)malloc(rows * E * sizeof(float));
  for (size_t li = 0; li < c->num_layers; li++) {
    const layer_t* L = &m->layers[li];
    /* model.rs:246-300 forward_layer */
    t0r_rmsnorm(x, L->norm, normed, rows, E, 1e-8f);
    if (!L->is_group) {
      mhsa(m, L, normed, v, p, tmask, ct, st, xt, tmp);
    } else {
      /* swap_dims(0,1): [v,p,e] -> [p,v,e] */
      for (size_t row = 0; row < v; row++)
        for (size_t pi = 0; pi < p; pi++) memcpy(tmp2 + (pi * v + row) * E, normed + (row * p + pi) * E, E * 4);
      mhsa(m, L, tmp2, p, v, gmask, NULL, NULL, NULL, normed);
      for (size_t row = 0; row < v; row++)
        for (size_t pi = 0; pi < p; pi++) memcpy(tmp + (row * p + pi) * E, normed + (pi * v + row) * E, E * 4);
    }
    for (size_t i = 0; i < rows * E; i++) x[i] = x[i] + tmp[i];
    t0r_rmsnorm(x, L->mlp_norm, normed, rows, E, 1e-8f);
    swiglu(m, L, normed, rows, tmp);
    for (size_t i = 0; i < rows * E; i++) x[i] = x[i] + tmp[i];
    if (li == 0 && tr_l0) memcpy(tr_l0, x, rows * E * sizeof(float));
  }
  t0r_rmsnorm(x, m->out_norm, normed, rows, E, 1e-8f);
  size_t nq = c->n_quantiles;
  float* dec = (float*)malloc(rows * ps * nq * sizeof(float));
  residual_block(&m->dec, normed, rows, dec);
  t0r_quantile_head(dec, out, rows * ps, nq);
  free(dec);
  free(normed);
  free(tmp);
  free(tmp2);
  free(ct);
  free(st);
  free(xt);
  free(tmask);
  free(gmask);
  free(pvt);
  free(pg);
  free(att);
  free(x);
  return T0R_OK;
}

int t0r_forward(const t0r_model* m, size_t v, size_t t, const float* variates, const int8_t* mask,
                const int64_t* group_ids, const int64_t* variate_type, float* out, float* tr_pe, float* tr_l0) {
  if (!m) return T0R_ERR_INVALID_ARG;
  series_t s = {v, t, (float*)variates, (int8_t*)mask, (int64_t*)group_ids, (int64_t*)variate_type};
  return forward_series(m, &s, out, tr_pe, tr_l0);
}

/* model.rs:448-531 forecast_series_prepare + finish (≡ t0-fast lib.rs:50-97) */
static int forecast_window(const t0r_model* m, const series_t* raw, size_t t_ctx, size_t horizon, float* out) {
  const t0r_config* c = &m->cfg;
  size_t ps = c->patch_size, nq = c->n_quantiles, v = raw->v;
  if (t_ctx == 0) return T0R_ERR_INVALID_ARG;
  size_t pad_left = (ps - t_ctx % ps) % ps;
  size_t padded_h = (horizon + ps - 1) / ps * ps;
  size_t padded_ctx = t_ctx + pad_left;
  if (padded_h > T0R_MAX_HORIZON) return T0R_ERR_HORIZON;
  series_t win;
  series_pad(raw, ps, t_ctx, &win);
  size_t n = v * win.t;
  float* scaled = (float*)malloc((n ? n : 1) * 4);
  float* loc = (float*)malloc((n ? n : 1) * 4);
  float* scl = (float*)malloc((n ? n : 1) * 4);
  int rc = t0r_scale_input(win.variates, win.mask, win.group_ids, win.variate_type, v, win.t, c->scaler_use_arcsinh,
                           c->scaler_eps, c->scaler_variance_offset, scaled, loc, scl);
  if (rc) {
    series_free(&win);
    free(scaled);
    free(loc);
    free(scl);
    return rc;
  }
  size_t p = win.t / ps;
  float* pred = (float*)malloc((v * p * ps * nq != 0 ? v * p * ps * nq : 1) * sizeof(float));
  series_t sc = {v, win.t, scaled, win.mask, win.group_ids, win.variate_type};
  rc = forward_series(m, &sc, pred, NULL, NULL);
  if (!rc) {
    /* scaler.rs:125-148 rescale_predictions */
    size_t per_row = p * ps * nq;
    for (size_t row = 0; row < v; row++)
      for (size_t pi = 0; pi < p; pi++) {
        size_t ti = row * win.t + pi * ps + (ps - 1);
        float l = loc[ti], s = scl[ti];
        size_t base = row * per_row + pi * ps * nq;
        for (size_t i = 0; i < ps * nq; i++) {
          float r = pred[base + i];
          float u = c->scaler_use_arcsinh ? sinhf(r) : r;
          pred[base + i] = u * s + l;
        }
      }
    /* slice patches [context_patches-1, +horizon_patches) then truncate to horizon */
    size_t ctx_p = padded_ctx / ps, hp = padded_h / ps, per_patch = ps * nq;
    for (size_t row = 0; row < v; row++)
      for (size_t h = 0; h < hp; h++) {
        size_t src = row * per_row + (ctx_p - 1 + h) * per_patch;
        for (size_t i = 0; i < per_patch; i++) {
          size_t step = h * ps + i / nq;
          if (step >= horizon) break;
          out[row * horizon * nq + h * per_patch + i] = pred[src + i];
        }
      }
  }
  free(pred);
  series_free(&win);
  free(scaled);
  free(loc);
  free(scl);
  return rc;
}

/* model.rs:322-333 forecast */
int t0r_forecast(const t0r_model* m, const float* ctx, size_t v, size_t t_ctx, size_t horizon, float* out) {
  if (!m || v == 0) return T0R_ERR_INVALID_ARG;
  series_t raw;
  from_context(ctx, v, t_ctx, horizon, &raw);
  int rc = forecast_window(m, &raw, t_ctx, horizon, out);
  series_free(&raw);
  return rc;
}

/* model.rs:385-407 forecast_batch_chunked (data.rs:96-105 from_context_batch) */
int t0r_forecast_batch_chunked(const t0r_model* m, const float* ctx, size_t n_signals, size_t t_ctx, size_t horizon,
                               size_t chunk, float* out) {
  if (!m) return T0R_ERR_INVALID_ARG;
  size_t nq = m->cfg.n_quantiles;
  chunk = (chunk == 0 || chunk > n_signals) ? n_signals : chunk;
  for (size_t start = 0; start < n_signals; start += chunk) {
    size_t n = chunk < n_signals - start ? chunk : n_signals - start;
    series_t raw;
    from_context(ctx + start * t_ctx, n, t_ctx, horizon, &raw);
    for (size_t row = 0; row < n; row++)
      for (size_t col = 0; col < raw.t; col++) raw.group_ids[row * raw.t + col] = (int64_t)row;
    int rc = forecast_window(m, &raw, t_ctx, horizon, out + start * horizon * nq);
    series_free(&raw);
    if (rc) return rc;
  }
  return T0R_OK;
}

/* crates/t0-fast/src/lib.rs:175-242 forecast_batch_rows_chunked_async */
int t0r_forecast_batch_rows_chunked(const t0r_model* m, const float* ctx, const size_t* lengths, size_t n_signals,
                                    size_t horizon, size_t chunk, float* out) {
  if (!m) return T0R_ERR_INVALID_ARG;
  size_t ps = m->cfg.patch_size, nq = m->cfg.n_quantiles;
  chunk = (chunk == 0 || chunk > n_signals) ? n_signals : chunk;
  size_t* offs = (size_t*)malloc((n_signals + 1) * sizeof(size_t));
  offs[0] = 0;
  for (size_t i = 0; i < n_signals; i++) offs[i + 1] = offs[i] + lengths[i];
  int rc = T0R_OK;
  for (size_t start = 0; start < n_signals && !rc; start += chunk) {
    size_t n = chunk < n_signals - start ? chunk : n_signals - start;
    size_t common = 0;
    for (size_t r = 0; r < n; r++) {
      size_t a = (lengths[start + r] + ps - 1) / ps * ps;
      if (a > common) common = a;
    }
    size_t t = common + horizon;
    series_t raw;
    series_alloc(&raw, n, t);
    for (size_t i = 0; i < n * t; i++) {
      raw.mask[i] = MT_PAD;
      raw.group_ids[i] = -1;
      raw.variate_type[i] = -1;
    }
    for (size_t r = 0; r < n; r++) {
      size_t len = lengths[start + r], lead = common - len;
      const float* src = ctx + offs[start + r];
      for (size_t col = 0; col < len; col++) {
        size_t idx = r * t + lead + col;
        if (isnan(src[col])) {
          raw.variates[idx] = 0.0f;
          raw.mask[idx] = MT_MISSING;
        } else {
          raw.variates[idx] = src[col];
          raw.mask[idx] = MT_VALID;
        }
        raw.group_ids[idx] = (int64_t)r;
        raw.variate_type[idx] = VT_TARGET;
      }
      for (size_t col = common; col < t; col++) {
        raw.group_ids[r * t + col] = (int64_t)r;
        raw.variate_type[r * t + col] = VT_TARGET;
        raw.mask[r * t + col] = MT_WITHHELD;
      }
    }
    rc = forecast_window(m, &raw, common, horizon, out + start * horizon * nq);
    series_free(&raw);
  }
  free(offs);
  return rc;
}

/* Multivariate batch with explicit per-row group ids (built from the pub
 * TimeSeries fields, data.rs:24-33, the way lib.rs:208-236 builds its rows). */
int t0r_forecast_grouped(const t0r_model* m, const float* ctx, const int64_t* row_group, size_t n_rows, size_t t_ctx,
                         size_t horizon, float* out) {
  if (!m || n_rows == 0) return T0R_ERR_INVALID_ARG;
  for (size_t r = 0; r < n_rows; r++)
    if (row_group[r] < 0) return T0R_ERR_INVALID_ARG;
  series_t raw;
  from_context(ctx, n_rows, t_ctx, horizon, &raw);
  for (size_t r = 0; r < n_rows; r++)
    for (size_t col = 0; col < raw.t; col++) raw.group_ids[r * raw.t + col] = row_group[r];
  int rc = forecast_window(m, &raw, t_ctx, horizon, out);
  series_free(&raw);
  return rc;
}

/* Autoregressive loop over forecast_grouped: each step appends every row's
 * median-level quantile and re-windows to the trailing t_ctx values.  out is
 * [n_rows, steps*horizon, n_q]. */
static size_t median_index(const t0r_config* c) {
  size_t best = 0;
  for (size_t i = 1; i < c->n_quantiles; i++)
    if (fabsf(c->quantile_levels[i] - 0.5f) < fabsf(c->quantile_levels[best] - 0.5f)) best = i;
  return best;
}

int t0r_forecast_grouped_ar(const t0r_model* m, const float* ctx, const int64_t* row_group, size_t n_rows,
                            size_t t_ctx, size_t horizon, size_t steps, float* out) {
  if (!m || n_rows == 0 || horizon == 0) return T0R_ERR_INVALID_ARG;
  size_t nq = m->cfg.n_quantiles, med = median_index(&m->cfg);
  float* win = (float*)malloc(n_rows * t_ctx * sizeof(float));
  memcpy(win, ctx, n_rows * t_ctx * sizeof(float));
  float* step_out = (float*)malloc(n_rows * horizon * nq * sizeof(float));
  int rc = T0R_OK;
  for (size_t s = 0; s < steps && !rc; s++) {
    rc = t0r_forecast_grouped(m, win, row_group, n_rows, t_ctx, horizon, step_out);
    if (rc) break;
    for (size_t r = 0; r < n_rows; r++) {
      memcpy(out + (r * steps * horizon + s * horizon) * nq, step_out + r * horizon * nq, horizon * nq * 4);
      float* w = win + r * t_ctx;
      if (horizon >= t_ctx) {
        for (size_t i = 0; i < t_ctx; i++) w[i] = step_out[(r * horizon + horizon - t_ctx + i) * nq + med];
      } else {
        memmove(w, w + horizon, (t_ctx - horizon) * sizeof(float));
        for (size_t i = 0; i < horizon; i++) w[t_ctx - horizon + i] = step_out[(r * horizon + i) * nq + med];
      }
    }
  }
  free(win);
  free(step_out);
  return rc;
}

/* model.rs:582-665 forecast_rollout (single univariate series) */
int t0r_forecast_rollout(const t0r_model* m, const float* ctx, size_t t_ctx, size_t prediction_length,
                         const float* query, size_t n_query, float* out) {
  if (!m || n_query == 0 || t_ctx == 0) return T0R_ERR_INVALID_ARG;
  const t0r_config* c = &m->cfg;
  size_t ps = c->patch_size, nt = c->n_quantiles;
  float trained_mass[T0R_MAX_QUANTILES];
  t0r_prob_mass(c->quantile_levels, nt, trained_mass);
  float* query_mass = (float*)malloc(n_query * sizeof(float));
  t0r_prob_mass(query, n_query, query_mass);
  size_t context_width = (t_ctx + ps - 1) / ps * ps;
  size_t horizon0 = (prediction_length + ps - 1) / ps * ps;
  if (horizon0 > T0R_MAX_HORIZON) horizon0 = T0R_MAX_HORIZON;
  float* block0 = (float*)malloc((horizon0 * nt != 0 ? horizon0 * nt : 1) * sizeof(float));
  int rc = t0r_forecast(m, ctx, 1, t_ctx, horizon0, block0);
  if (rc) {
    free(block0);
    free(query_mass);
    return rc;
  }
  /* out chunks are written straight into `out` (truncated to prediction_length) */
  float* first = (float*)malloc((horizon0 * n_query != 0 ? horizon0 * n_query : 1) * sizeof(float));
  for (size_t h = 0; h < horizon0; h++)
    t0r_interpolate_quantiles(query, n_query, c->quantile_levels, block0 + h * nt, nt, first + h * n_query);
  free(block0);
  size_t written = 0;
  size_t take = horizon0 < prediction_length ? horizon0 : prediction_length;
  memcpy(out, first, take * n_query * sizeof(float));
  written = take;
  if (prediction_length <= horizon0) {
    free(first);
    free(query_mass);
    return T0R_OK;
  }
  size_t n_paths = n_query;
  size_t buf_cap = t_ctx + prediction_length + T0R_MAX_HORIZON + ps;
  float* paths = (float*)malloc(n_paths * buf_cap * sizeof(float));
  size_t buf_len = t_ctx;
  for (size_t j = 0; j < n_paths; j++) memcpy(paths + j * buf_cap, ctx, t_ctx * sizeof(float));
  size_t remaining = prediction_length - horizon0;
  float* prev = first;
  size_t prev_width = horizon0;
  float* wts = (float*)malloc(n_paths * nt * sizeof(float));
  float* smp = (float*)malloc(n_paths * nt * sizeof(float));
  for (size_t j = 0; j < n_paths; j++)
    for (size_t pq = 0; pq < nt; pq++) wts[j * nt + pq] = trained_mass[pq] * query_mass[j];
  while (remaining > 0 && !rc) {
    for (size_t j = 0; j < n_paths; j++)
      for (size_t h = 0; h < prev_width; h++) paths[j * buf_cap + buf_len + h] = prev[h * n_query + j];
    buf_len += prev_width;
    size_t horizon = (remaining + ps - 1) / ps * ps;
    if (horizon > T0R_MAX_HORIZON) horizon = T0R_MAX_HORIZON;
    float* bctx = (float*)calloc(n_paths * context_width, sizeof(float));
    for (size_t j = 0; j < n_paths; j++) {
      size_t wl = context_width < buf_len ? context_width : buf_len;
      memcpy(bctx + j * context_width + (context_width - wl), paths + j * buf_cap + buf_len - wl, wl * sizeof(float));
    }
    float* blocks = (float*)malloc(n_paths * horizon * nt * sizeof(float));
    rc = t0r_forecast_batch_chunked(m, bctx, n_paths, context_width, horizon, 16, blocks);
    free(bctx);
    if (rc) {
      free(blocks);
      break;
    }
    float* reduced = (float*)malloc(horizon * n_query * sizeof(float));
    for (size_t h = 0; h < horizon; h++) {
      for (size_t j = 0; j < n_paths; j++)
        for (size_t pq = 0; pq < nt; pq++) smp[j * nt + pq] = blocks[j * horizon * nt + h * nt + pq];
      t0r_weighted_quantile(query, n_query, wts, smp, n_paths * nt, reduced + h * n_query);
    }
    free(blocks);
    size_t room = prediction_length - written;
    take = horizon < room ? horizon : room;
    memcpy(out + written * n_query, reduced, take * n_query * sizeof(float));
    written += take;
    /* buffers must hold the next append */
    if (buf_len + horizon > buf_cap) {
      size_t keep = context_width;
      for (size_t j = 0; j < n_paths; j++)
        memmove(paths + j * buf_cap, paths + j * buf_cap + buf_len - keep, keep * sizeof(float));
      buf_len = keep;
    }
    free(prev);
    prev = reduced;
    prev_width = horizon;
    remaining = remaining > horizon ? remaining - horizon : 0; /* saturating_sub, model.rs:660 */
  }
  free(prev);
  free(paths);
  free(wts);
  free(smp);
  free(query_mass);
  return rc;
}
