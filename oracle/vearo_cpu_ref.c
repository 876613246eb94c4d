/*
 * vearo_cpu_ref.c -- CPU oracle (TEST INFRASTRUCTURE ONLY; see vearo_cpu_ref.h).
 *
 * A restatement, in plain C, of the hot-path functions of vearo-backend-cpu and
 * of the autograd arms that compose them. Each function cites the Rust lines it
 * follows. Loop order, accumulation order and the f32 rounding points are kept;
 * the per-element coordinate Vec allocations of the Rust code are not (they do
 * not affect results). Build flags: -O2 -ffp-contract=off (no fast-math).
 */
#include "vearo_cpu_ref.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ helpers */

static int panicf(char* err, size_t errlen, const char* fmt, ...) {
  if (err && errlen) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
  }
  return VO_PANIC;
}

void vo_contiguous_layout(vo_layout* l, int rank, const int64_t* dims) {
  int64_t acc = 1;
  l->rank = rank;
  for (int i = rank - 1; i >= 0; --i) {
    l->dims[i] = dims[i];
    l->strides[i] = acc;
    acc *= dims[i];
  }
}

static int64_t numel_of(const vo_layout* l) {
  int64_t n = 1;
  for (int i = 0; i < l->rank; ++i) n *= l->dims[i];
  return n;
}

/* Tensor::is_contiguous (tensor.rs:335-337): strides equal the row-major strides. */
static int is_contig(const vo_layout* l) {
  int64_t acc = 1;
  for (int i = l->rank - 1; i >= 0; --i) {
    if (l->strides[i] != acc) return 0;
    acc *= l->dims[i];
  }
  return 1;
}

/* get_offset (shape.rs:268-281): trailing-aligned coordinate, size-1 dims broadcast. */
static int64_t get_offset(const int64_t* coord, int coord_len, const vo_layout* l) {
  int64_t off = 0;
  int co = coord_len - l->rank;
  if (co < 0) co = 0;
  for (int i = 0; i < l->rank; ++i) {
    int64_t c = l->dims[i] == 1 ? 0 : coord[co + i];
    off += c * l->strides[i];
  }
  return off;
}

/* flat_to_coord (cpu:655-663) followed by get_offset; identity on contiguous layouts. */
static int64_t flat_offset(int64_t flat, const vo_layout* l, int contig) {
  if (contig) return flat;
  int64_t coord[VO_MAX_RANK];
  for (int i = l->rank - 1; i >= 0; --i) {
    coord[i] = flat % l->dims[i];
    flat /= l->dims[i];
  }
  return get_offset(coord, l->rank, l);
}

/* NdIterator::step (shape.rs:240-264). Returns 0 when exhausted. */
static int nd_step(int64_t* coord, const int64_t* dims, int rank) {
  if (rank == 0) return 0;
  int idx = rank - 1;
  for (;;) {
    coord[idx] += 1;
    if (coord[idx] < dims[idx]) return 1;
    coord[idx] = 0;
    if (idx == 0) return 0;
    idx -= 1;
  }
}

/* Shape::broadcast (shape.rs:91-124). Returns 0 if not broadcastable. */
static int broadcast_shape(const vo_layout* a, const vo_layout* b, vo_layout* out) {
  int r = a->rank > b->rank ? a->rank : b->rank;
  if (r > VO_MAX_RANK) return 0;
  out->rank = r;
  for (int i = 0; i < r; ++i) {
    int64_t ad = i < a->rank ? a->dims[a->rank - 1 - i] : 1;
    int64_t bd = i < b->rank ? b->dims[b->rank - 1 - i] : 1;
    int64_t od;
    if (ad == bd) od = ad;
    else if (ad == 1) od = bd;
    else if (bd == 1) od = ad;
    else return 0;
    out->dims[r - 1 - i] = od;
  }
  vo_contiguous_layout(out, r, out->dims);
  return 1;
}

/* Rust `{}` Display of f32: the shortest digit string that round-trips, printed
 * positionally (Rust never switches to exponent form for Display). */
void vo_format_f32(float v, char* buf, size_t len) {
  if (isnan(v)) { snprintf(buf, len, "NaN"); return; }
  if (isinf(v)) { snprintf(buf, len, v < 0 ? "-inf" : "inf"); return; }
  if (v == 0.0f) { snprintf(buf, len, signbit(v) ? "-0" : "0"); return; }
  char sci[64];
  int prec;
  for (prec = 0; prec < 9; ++prec) {
    snprintf(sci, sizeof sci, "%.*e", prec, (double)v);
    if (strtof(sci, NULL) == v) break;
  }
  /* sci = [-]d[.ddd]e[+-]XX */
  const char* p = sci;
  int neg = 0;
  if (*p == '-') { neg = 1; ++p; }
  char digits[32];
  int nd = 0;
  while (*p && *p != 'e') {
    if (*p != '.') digits[nd++] = *p;
    ++p;
  }
  int exp10 = atoi(p + 1); /* value = 0.d1d2.. * 10^(exp10+1) */
  while (nd > 1 && digits[nd - 1] == '0') --nd;
  char out[96];
  int o = 0;
  if (neg) out[o++] = '-';
  int point = exp10 + 1; /* digits before the decimal point */
  if (point <= 0) {
    out[o++] = '0';
    out[o++] = '.';
    for (int i = 0; i < -point; ++i) out[o++] = '0';
    for (int i = 0; i < nd; ++i) out[o++] = digits[i];
  } else {
    for (int i = 0; i < point; ++i) out[o++] = i < nd ? digits[i] : '0';
    if (nd > point) {
      out[o++] = '.';
      for (int i = point; i < nd; ++i) out[o++] = digits[i];
    }
  }
  out[o] = 0;
  snprintf(buf, len, "%s", out);
}

/* `value.round() as usize` in Rust: round half away from zero, saturating cast. */
static uint64_t round_to_usize(float v) {
  float r = roundf(v);
  if (!(r > 0.0f)) return 0; /* NaN and non-positive saturate to 0 */
  if ((double)r >= 18446744073709551616.0) return UINT64_MAX;
  return (uint64_t)r;
}

/* --------------------------------------------------------- elementwise ops */

/* elementwise_op (cpu:160-202) with add/sub/mul/div closures (cpu:204-238). */
int vo_binary(int op, const float* lhs, const vo_layout* ll, const float* rhs,
              const vo_layout* rl, float* out, const vo_layout* out_shape, char* err,
              size_t errlen) {
  vo_layout bs;
  if (!broadcast_shape(ll, rl, &bs)) return panicf(err, errlen, "Shapes are not broadcastable");
  if (bs.rank != out_shape->rank) return panicf(err, errlen, "output shape mismatch");
  for (int i = 0; i < bs.rank; ++i)
    if (bs.dims[i] != out_shape->dims[i]) return panicf(err, errlen, "output shape mismatch");
  int64_t n = numel_of(&bs);
  if (n == 0) return VO_OK;
  int same = ll->rank == rl->rank;
  for (int i = 0; same && i < ll->rank; ++i) same = ll->dims[i] == rl->dims[i];
  if (is_contig(ll) && is_contig(rl) && same) {
    for (int64_t i = 0; i < n; ++i) {
      float a = lhs[i], b = rhs[i];
      out[i] = op == 0 ? a + b : op == 1 ? a - b : op == 2 ? a * b : a / b;
    }
    return VO_OK;
  }
  int64_t coord[VO_MAX_RANK] = {0};
  int64_t i = 0;
  do {
    float a = lhs[get_offset(coord, bs.rank, ll)];
    float b = rhs[get_offset(coord, bs.rank, rl)];
    out[i++] = op == 0 ? a + b : op == 1 ? a - b : op == 2 ? a * b : a / b;
  } while (nd_step(coord, bs.dims, bs.rank));
  return VO_OK;
}

/* gelu (cpu:458-497): tanh approximation with f32 constants 0.797_884_56 and 0.044_715. */
static inline float gelu1(float v) {
  const float SQRT_2_OVER_PI = 0.79788456f;
  const float COEFF = 0.044715f;
  float v3 = v * v * v;
  float inner = SQRT_2_OVER_PI * (v + COEFF * v3);
  return 0.5f * v * (1.0f + tanhf(inner));
}

void vo_gelu(const float* x, const vo_layout* xl, float* out) {
  int64_t n = numel_of(xl);
  if (n == 0) return;
  int contig = is_contig(xl);
  if (contig) {
    for (int64_t i = 0; i < n; ++i) out[i] = gelu1(x[i]);
    return;
  }
  int64_t coord[VO_MAX_RANK] = {0};
  int64_t i = 0;
  do {
    out[i++] = gelu1(x[get_offset(coord, xl->rank, xl)]);
  } while (nd_step(coord, xl->dims, xl->rank));
}

/* gelu_grad_mask (autograd:383-403), evaluated on the contiguous copy of x. */
static inline float gelu_mask1(float v) {
  const float SQRT_2_OVER_PI = 0.79788456f;
  const float COEFF = 0.044715f;
  const float DERIV_COEFF = 0.134145f;
  float v3 = v * v * v;
  float inner = SQRT_2_OVER_PI * (v + COEFF * v3);
  float t = tanhf(inner);
  float t_sq = t * t;
  float sech_sq = 1.0f - t_sq;
  float inner_deriv = SQRT_2_OVER_PI * (1.0f + DERIV_COEFF * v * v);
  return 0.5f * (1.0f + t) + 0.5f * v * sech_sq * inner_deriv;
}

void vo_gelu_grad_mask(const float* x, int64_t n, float* mask) {
  for (int64_t i = 0; i < n; ++i) mask[i] = gelu_mask1(x[i]);
}

/* ----------------------------------------------------------------- softmax */

/* softmax (cpu:501-563): per reduced coordinate, max (strict >, from -inf),
 * sequential sum of exp(v-max), then exp(v-max)/sum written row-major. */
int vo_softmax(const float* x, const vo_layout* xl, int dim, float* out, char* err,
               size_t errlen) {
  int rank = xl->rank;
  if (dim < 0 || dim >= rank) return panicf(err, errlen, "Softmax dim out of range");
  int64_t n = numel_of(xl);
  if (n == 0) return VO_OK;
  int64_t dsz = xl->dims[dim];
  vo_layout red = *xl;
  red.dims[dim] = 1;
  vo_layout oc;
  vo_contiguous_layout(&oc, rank, xl->dims);
  int64_t coord[VO_MAX_RANK] = {0};
  do {
    int64_t c[VO_MAX_RANK];
    memcpy(c, coord, sizeof c);
    float max_val = -INFINITY;
    for (int64_t d = 0; d < dsz; ++d) {
      c[dim] = d;
      float v = x[get_offset(c, rank, xl)];
      if (v > max_val) max_val = v;
    }
    float sum_exp = 0.0f;
    for (int64_t d = 0; d < dsz; ++d) {
      c[dim] = d;
      float v = x[get_offset(c, rank, xl)];
      sum_exp += expf(v - max_val);
    }
    for (int64_t d = 0; d < dsz; ++d) {
      c[dim] = d;
      float v = x[get_offset(c, rank, xl)];
      out[get_offset(c, rank, &oc)] = expf(v - max_val) / sum_exp;
    }
  } while (nd_step(coord, red.dims, rank));
  return VO_OK;
}

/* -------------------------------------------------------------- reductions */

/* reduce_sum_data (cpu:585-620): row-major walk over the input, each output
 * element receives its contributions in increasing dim-index order. */
static int reduce_sum(const float* x, const vo_layout* xl, int dim, int keep_dim,
                      float* out, char* err, size_t errlen) {
  int rank = xl->rank;
  if (dim < 0 || dim >= rank) return panicf(err, errlen, "Reduction dim out of range");
  int64_t out_numel = 1;
  for (int i = 0; i < rank; ++i)
    if (i != dim) out_numel *= xl->dims[i];
  for (int64_t i = 0; i < out_numel; ++i) out[i] = 0.0f;
  int64_t n = numel_of(xl);
  if (n == 0) return VO_OK;
  int64_t coord[VO_MAX_RANK] = {0};
  (void)keep_dim; /* keep_dim only changes the output shape, not its flat order */
  do {
    int64_t idx = 0, stride = 1;
    for (int d = rank - 1; d >= 0; --d) {
      if (d == dim) continue;
      idx += coord[d] * stride;
      stride *= xl->dims[d];
    }
    out[idx] += x[get_offset(coord, rank, xl)];
  } while (nd_step(coord, xl->dims, rank));
  return VO_OK;
}

int vo_sum(const float* x, const vo_layout* xl, int dim, int keep_dim, float* out,
           char* err, size_t errlen) {
  return reduce_sum(x, xl, dim, keep_dim, out, err, errlen);
}

/* mean (cpu:641-653): the sum, then one division per output by the axis length. */
int vo_mean(const float* x, const vo_layout* xl, int dim, int keep_dim, float* out,
            char* err, size_t errlen) {
  int rc = reduce_sum(x, xl, dim, keep_dim, out, err, errlen);
  if (rc) return rc;
  float count = (float)xl->dims[dim];
  int64_t out_numel = 1;
  for (int i = 0; i < xl->rank; ++i)
    if (i != dim) out_numel *= xl->dims[i];
  for (int64_t i = 0; i < out_numel; ++i) out[i] /= count;
  return VO_OK;
}

/* --------------------------------------------------------------- layernorm */

static int ln_checks(const vo_layout* xl, const vo_layout* wl, const vo_layout* bl,
                     char* err, size_t errlen) {
  if (xl->rank < 1) return panicf(err, errlen, "LayerNorm input must be at least rank 1");
  int64_t C = xl->dims[xl->rank - 1];
  if (wl->rank != 1) return panicf(err, errlen, "LayerNorm weight must be rank 1");
  if (bl->rank != 1) return panicf(err, errlen, "LayerNorm bias must be rank 1");
  if (wl->dims[0] != C) return panicf(err, errlen, "Weight dimension must match norm_dim");
  if (bl->dims[0] != C) return panicf(err, errlen, "Bias dimension must match norm_dim");
  return VO_OK;
}

/* layernorm (cpu:665-740). */
int vo_layernorm(const float* x, const vo_layout* xl, const float* w, const vo_layout* wl,
                 const float* b, const vo_layout* bl, float eps, float* out, char* err,
                 size_t errlen) {
  if (numel_of(xl) == 0) return VO_OK;
  int rc = ln_checks(xl, wl, bl, err, errlen);
  if (rc) return rc;
  int64_t C = xl->dims[xl->rank - 1];
  int64_t outer = numel_of(xl) / C;
  int xc = is_contig(xl);
  for (int64_t r = 0; r < outer; ++r) {
    int64_t base = r * C;
    float sum = 0.0f;
    for (int64_t i = 0; i < C; ++i) sum += x[flat_offset(base + i, xl, xc)];
    float mean = sum / (float)C;
    float sum_sq = 0.0f;
    for (int64_t i = 0; i < C; ++i) {
      float diff = x[flat_offset(base + i, xl, xc)] - mean;
      sum_sq += diff * diff;
    }
    float var = sum_sq / (float)C;
    float inv_std = 1.0f / sqrtf(var + eps);
    for (int64_t i = 0; i < C; ++i) {
      float x_hat = (x[flat_offset(base + i, xl, xc)] - mean) * inv_std;
      out[base + i] = x_hat * w[i * wl->strides[0]] + b[i * bl->strides[0]];
    }
  }
  return VO_OK;
}

/* layernorm_backward (cpu:742-858). gw/gb accumulate across rows in ascending
 * row order; dx uses (C*go*w - sum_go_w - x_hat*sum_go_w_xhat)*inv_std/C. */
int vo_layernorm_backward(const float* x, const vo_layout* xl, const float* w,
                          const vo_layout* wl, const vo_layout* bl, const float* go,
                          const vo_layout* gol, float eps, float* gx, float* gw, float* gb,
                          char* err, size_t errlen) {
  int64_t n = numel_of(xl);
  for (int64_t i = 0; i < numel_of(wl); ++i) gw[i] = 0.0f;
  for (int64_t i = 0; i < numel_of(bl); ++i) gb[i] = 0.0f;
  if (n == 0) return VO_OK;
  int rc = ln_checks(xl, wl, bl, err, errlen);
  if (rc) return rc;
  int64_t C = xl->dims[xl->rank - 1];
  int64_t outer = n / C;
  int xc = is_contig(xl);
  int gc = is_contig(gol) && gol->rank == xl->rank;
  float Cf = (float)C;
  for (int64_t r = 0; r < outer; ++r) {
    int64_t base = r * C;
    float sum = 0.0f;
    for (int64_t i = 0; i < C; ++i) sum += x[flat_offset(base + i, xl, xc)];
    float mean = sum / Cf;
    float sum_sq = 0.0f;
    for (int64_t i = 0; i < C; ++i) {
      float diff = x[flat_offset(base + i, xl, xc)] - mean;
      sum_sq += diff * diff;
    }
    float var = sum_sq / Cf;
    float inv_std = 1.0f / sqrtf(var + eps);
    float sum_go_w = 0.0f, sum_go_w_xhat = 0.0f;
    for (int64_t i = 0; i < C; ++i) {
      float go_val = go[gc ? base + i : flat_offset(base + i, gol, 0)];
      float x_hat = (x[flat_offset(base + i, xl, xc)] - mean) * inv_std;
      float w_val = w[i * wl->strides[0]];
      sum_go_w += go_val * w_val;
      sum_go_w_xhat += go_val * w_val * x_hat;
      gw[i] += go_val * x_hat;
      gb[i] += go_val;
    }
    for (int64_t i = 0; i < C; ++i) {
      float go_val = go[gc ? base + i : flat_offset(base + i, gol, 0)];
      float x_hat = (x[flat_offset(base + i, xl, xc)] - mean) * inv_std;
      float w_val = w[i * wl->strides[0]];
      float term1 = Cf * go_val * w_val;
      float term2 = sum_go_w;
      float term3 = x_hat * sum_go_w_xhat;
      gx[base + i] = (term1 - term2 - term3) * inv_std / Cf;
    }
  }
  return VO_OK;
}

/* --------------------------------------------------------------- embedding */

static int check_token(float tv, int64_t vocab, uint64_t* tok, char* err, size_t errlen) {
  char buf[64];
  if (!(tv >= 0.0f)) {
    vo_format_f32(tv, buf, sizeof buf);
    return panicf(err, errlen, "Token ID cannot be negative: %s", buf);
  }
  *tok = round_to_usize(tv);
  if (*tok >= (uint64_t)vocab)
    return panicf(err, errlen, "Token ID %llu out of vocabulary bound %lld",
                  (unsigned long long)*tok, (long long)vocab);
  return VO_OK;
}

/* embedding (cpu:860-918): out[i, d] = W[round(ids[i]), d], a pure copy. */
int vo_embedding(const float* ids, const vo_layout* il, const float* w, const vo_layout* wl,
                 float* out, char* err, size_t errlen) {
  if (wl->rank != 2) return panicf(err, errlen, "Weight must be rank 2 (vocab_size, embedding_dim)");
  int64_t V = wl->dims[0], D = wl->dims[1];
  int64_t n = numel_of(il);
  if (n == 0) return VO_OK;
  int ic = is_contig(il);
  for (int64_t i = 0; i < n; ++i) {
    uint64_t tok;
    int rc = check_token(ids[flat_offset(i, il, ic)], V, &tok, err, errlen);
    if (rc) return rc;
    for (int64_t d = 0; d < D; ++d)
      out[i * D + d] = w[(int64_t)tok * wl->strides[0] + d * wl->strides[1]];
  }
  return VO_OK;
}

/* embedding_backward (cpu:920-980): dense dW, dW[tok] += dy[i] for i ascending. */
int vo_embedding_backward(const float* ids, const vo_layout* il, const vo_layout* wl,
                          const float* go, const vo_layout* gol, float* gw, char* err,
                          size_t errlen) {
  if (wl->rank != 2) return panicf(err, errlen, "Weight must be rank 2 (vocab_size, embedding_dim)");
  int64_t V = wl->dims[0], D = wl->dims[1];
  int ok = gol->rank == il->rank + 1;
  for (int i = 0; ok && i < il->rank; ++i) ok = gol->dims[i] == il->dims[i];
  if (ok) ok = gol->dims[il->rank] == D;
  if (!ok) return panicf(err, errlen, "grad_out shape must be x.shape() + [embedding_dim]");
  for (int64_t i = 0; i < V * D; ++i) gw[i] = 0.0f;
  int64_t n = numel_of(il);
  int ic = is_contig(il), gc = is_contig(gol);
  for (int64_t i = 0; i < n; ++i) {
    uint64_t tok;
    int rc = check_token(ids[flat_offset(i, il, ic)], V, &tok, err, errlen);
    if (rc) return rc;
    for (int64_t d = 0; d < D; ++d)
      gw[(int64_t)tok * D + d] += go[flat_offset(i * D + d, gol, gc)];
  }
  return VO_OK;
}

/* ----------------------------------------------------------- cross entropy */

static int ce_checks(const vo_layout* ll, const vo_layout* tl, char* err, size_t errlen) {
  if (ll->rank != 2) return panicf(err, errlen, "Logits must be rank 2 (batch_size, vocab_size)");
  if (tl->rank != 1) return panicf(err, errlen, "Targets must be rank 1 (batch_size)");
  if (ll->dims[0] <= 0) return panicf(err, errlen, "Batch size must be greater than 0");
  if (tl->dims[0] != ll->dims[0]) return panicf(err, errlen, "Targets shape must match batch size");
  return VO_OK;
}

static int check_target(float tv, int64_t vocab, uint64_t* cls, char* err, size_t errlen) {
  char buf[64];
  if (!(tv >= 0.0f)) {
    vo_format_f32(tv, buf, sizeof buf);
    return panicf(err, errlen, "Target class cannot be negative: %s", buf);
  }
  *cls = round_to_usize(tv);
  if (*cls >= (uint64_t)vocab)
    return panicf(err, errlen, "Target class %llu out of vocab bounds %lld",
                  (unsigned long long)*cls, (long long)vocab);
  return VO_OK;
}

/* cross_entropy (cpu:982-1051): loss_sum -= (logit[t] - max - ln(sum_exp)) over
 * rows in order, returned as loss_sum / B. */
int vo_cross_entropy(const float* logits, const vo_layout* ll, const float* tgt,
                     const vo_layout* tl, float* loss, char* err, size_t errlen) {
  int rc = ce_checks(ll, tl, err, errlen);
  if (rc) return rc;
  int64_t B = ll->dims[0], V = ll->dims[1];
  int64_t ls0 = ll->strides[0], ls1 = ll->strides[1];
  float loss_sum = 0.0f;
  for (int64_t b = 0; b < B; ++b) {
    uint64_t t;
    rc = check_target(tgt[b * tl->strides[0]], V, &t, err, errlen);
    if (rc) return rc;
    const float* row = logits + b * ls0;
    float max_logit = -INFINITY;
    for (int64_t c = 0; c < V; ++c)
      if (row[c * ls1] > max_logit) max_logit = row[c * ls1];
    float sum_exp = 0.0f;
    for (int64_t c = 0; c < V; ++c) sum_exp += expf(row[c * ls1] - max_logit);
    float target_logit = row[(int64_t)t * ls1];
    float log_softmax = target_logit - max_logit - logf(sum_exp);
    loss_sum -= log_softmax;
  }
  *loss = loss_sum / (float)B;
  return VO_OK;
}

/* cross_entropy_backward (cpu:1053-1127): go * (p - 1[c==t]) / B. */
int vo_cross_entropy_backward(const float* logits, const vo_layout* ll, const float* tgt,
                              const vo_layout* tl, const float* grad_out,
                              int64_t grad_out_numel, float* gl, char* err, size_t errlen) {
  int rc = ce_checks(ll, tl, err, errlen);
  if (rc) return rc;
  if (grad_out_numel != 1) return panicf(err, errlen, "grad_out must be a scalar");
  int64_t B = ll->dims[0], V = ll->dims[1];
  int64_t ls0 = ll->strides[0], ls1 = ll->strides[1];
  float go_val = grad_out[0];
  float Bf = (float)B;
  for (int64_t b = 0; b < B; ++b) {
    uint64_t t;
    rc = check_target(tgt[b * tl->strides[0]], V, &t, err, errlen);
    if (rc) return rc;
    const float* row = logits + b * ls0;
    float max_logit = -INFINITY;
    for (int64_t c = 0; c < V; ++c)
      if (row[c * ls1] > max_logit) max_logit = row[c * ls1];
    float sum_exp = 0.0f;
    for (int64_t c = 0; c < V; ++c) sum_exp += expf(row[c * ls1] - max_logit);
    for (int64_t c = 0; c < V; ++c) {
      float p_c = expf(row[c * ls1] - max_logit) / sum_exp;
      float ind = (uint64_t)c == t ? 1.0f : 0.0f;
      gl[b * V + c] = go_val * (p_c - ind) / Bf;
    }
  }
  return VO_OK;
}

/* ----------------------------------------------------- autograd composites */

/* reduce_to (autograd:316-361): sum a contiguous gradient into target_shape,
 * trailing dims aligned, size-1 target dims collapsed, row-major order. */
int vo_reduce_to(const float* grad, const vo_layout* gshape, const int64_t* target,
                 int target_rank, float* out, char* err, size_t errlen) {
  int64_t out_numel = 1;
  for (int i = 0; i < target_rank; ++i) out_numel *= target[i];
  int same = gshape->rank == target_rank;
  for (int i = 0; same && i < target_rank; ++i) same = gshape->dims[i] == target[i];
  int64_t n = numel_of(gshape);
  if (same) {
    memcpy(out, grad, (size_t)n * sizeof(float));
    return VO_OK;
  }
  for (int64_t i = 0; i < out_numel; ++i) out[i] = 0.0f;
  if (n == 0) return VO_OK;
  if (gshape->rank < target_rank)
    return panicf(err, errlen, "Grad rank %d must be >= target rank %d", gshape->rank, target_rank);
  int64_t coord[VO_MAX_RANK] = {0};
  int64_t i = 0;
  do {
    int64_t tidx = 0, stride = 1;
    for (int d = target_rank - 1; d >= 0; --d) {
      int gd = gshape->rank - target_rank + d;
      int64_t c = target[d] == 1 ? 0 : coord[gd];
      tidx += c * stride;
      stride *= target[d];
    }
    out[tidx] += grad[i++];
  } while (nd_step(coord, gshape->dims, gshape->rank));
  return VO_OK;
}

/* The Softmax arm (autograd:547-553) as the five CPU ops it dispatches:
 * softmax, mul, sum(dim, keep=true), sub (broadcast), mul. */
int vo_softmax_backward_composite(const float* x, const float* dy, const vo_layout* xl,
                                  int dim, float* dx, char* err, size_t errlen) {
  int64_t n = numel_of(xl);
  if (n == 0) return VO_OK;
  float* y = (float*)malloc((size_t)n * sizeof(float));
  float* p = (float*)malloc((size_t)n * sizeof(float));
  float* t = (float*)malloc((size_t)n * sizeof(float));
  int64_t rd[VO_MAX_RANK];
  for (int i = 0; i < xl->rank; ++i) rd[i] = xl->dims[i];
  rd[dim] = 1;
  vo_layout sl;
  vo_contiguous_layout(&sl, xl->rank, rd);
  float* s = (float*)malloc((size_t)(n / (xl->dims[dim] ? xl->dims[dim] : 1) + 1) * sizeof(float));
  vo_layout cl;
  vo_contiguous_layout(&cl, xl->rank, xl->dims);
  int rc = vo_softmax(x, xl, dim, y, err, errlen);
  if (!rc) rc = vo_binary(2, dy, &cl, y, &cl, p, &cl, err, errlen);
  if (!rc) rc = vo_sum(p, &cl, dim, 1, s, err, errlen);
  if (!rc) rc = vo_binary(1, dy, &cl, s, &sl, t, &cl, err, errlen);
  if (!rc) rc = vo_binary(2, y, &cl, t, &cl, dx, &cl, err, errlen);
  free(y);
  free(p);
  free(t);
  free(s);
  return rc;
}

/* Linear bias add (cpu:183-196 broadcast branch) followed by gelu (cpu:469-477). */
void vo_gelu_bias_forward(const float* x, const float* bias, int64_t rows, int64_t C,
                          float* y) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < C; ++c) y[r * C + c] = gelu1(x[r * C + c] + bias[c]);
}

/* Gelu arm then Add arm: dh = dy * gelu_mask(x + bias) (autograd:542-546,
 * cpu:227-229), dbias = reduce_to(dh, [C]) (autograd:316-361, row-major sum). */
void vo_gelu_bias_backward(const float* x, const float* bias, const float* dy,
                           int64_t rows, int64_t C, float* dx, float* dbias) {
  for (int64_t c = 0; c < C; ++c) dbias[c] = 0.0f;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < C; ++c) {
      float h = x[r * C + c] + bias[c];
      float g = dy[r * C + c] * gelu_mask1(h);
      dx[r * C + c] = g;
      dbias[c] += g;
    }
}

/* ---------------------------------------------------------- libm probe */
void vo_math(int which, const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = which == 0 ? expf(x[i]) : which == 1 ? logf(x[i]) : tanhf(x[i]);
}
