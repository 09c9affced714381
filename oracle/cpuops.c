/*
 * cpuops.c -- TEST INFRASTRUCTURE ONLY. A plain-C restatement of Roost's CPU reference ops (CpuOps, C#) for the
 * attention + Gated DeltaNet path, used as the parity oracle by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg. Nothing in the product library links, calls or falls back to this code.
 *
 * Each function follows the reference source it cites, line for line in meaning: every element is widened to double,
 * all arithmetic is double, and each output element is rounded once into its element type (round to nearest even;
 * bf16 through round-to-odd to float first so the two roundings act as one). Where CpuOps throws an ArgumentException
 * before writing, these functions return a non-zero code before writing and leave a message in oracle_last_error().
 *
 * Parity pinning (which check pins which function) is listed in tests/test_oracle.py.
 */
#define _GNU_SOURCE
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { DT_F32 = 1, DT_F16 = 2, DT_BF16 = 3, DT_F64 = 4, DT_I32 = 10, DT_I64 = 12 };

static char g_err[512];
const char* oracle_last_error(void) { return g_err; }
static int fail(const char* msg) {
  snprintf(g_err, sizeof g_err, "%s", msg);
  return 1;
}

/* ---- Elements (reference: src/Starlings.Roost.Ops/CpuElements.cs:28-79, 128-160) ---- */

static float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_from_f32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* double -> bf16: NaN -> 0x7FC0, +-inf kept; otherwise round to float with round-to-odd, then to bf16 with RNE. */
uint16_t oracle_to_bf16(double v) {
  if (isnan(v)) return 0x7FC0;
  if (isinf(v)) return v > 0 ? 0x7F80 : 0xFF80;
  float f = (float)v;
  if (!isinf(f) && (double)f != v) {
    uint32_t bits = bits_from_f32(f);
    if ((bits & 1u) == 0) {
      bits += fabs((double)f) < fabs(v) ? 1 : (uint32_t)-1;
      f = f32_from_bits(bits);
    }
  }
  uint32_t u = bits_from_f32(f);
  if (isinf(f)) return (uint16_t)(u >> 16);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

double oracle_from_bf16(uint16_t b) { return (double)f32_from_bits((uint32_t)b << 16); }

static double load(const void* p, int dt, int64_t i) {
  switch (dt) {
    case DT_F32: return ((const float*)p)[i];
    case DT_F64: return ((const double*)p)[i];
    case DT_BF16: return oracle_from_bf16(((const uint16_t*)p)[i]);
    default: return NAN;
  }
}

static void store(void* p, int dt, int64_t i, double v) {
  switch (dt) {
    case DT_F32: ((float*)p)[i] = (float)v; break;
    case DT_F64: ((double*)p)[i] = v; break;
    case DT_BF16: ((uint16_t*)p)[i] = oracle_to_bf16(v); break;
    default: break;
  }
}

static int elem_size(int dt) { return dt == DT_F64 || dt == DT_I64 ? 8 : (dt == DT_F32 || dt == DT_I32 ? 4 : 2); }

/* ---- PagedAttention (reference: src/Starlings.Roost.Ops/CpuOps.cs:198-351) ---- */

typedef struct {
  int64_t q0, n, p0, kv_len;
} Seq;

static int attention_sequence(const int32_t* q_indptr, const int32_t* kv_indptr, const int32_t* last_len,
                              int64_t kv_indices_len, int b, int tokens, int page_size, int causal, Seq* s) {
  /* CpuOps.cs:300-335 AttentionSequence */
  int64_t q0 = q_indptr[b], q1 = q_indptr[b + 1], p0 = kv_indptr[b], p1 = kv_indptr[b + 1];
  int64_t pages = p1 - p0, n = q1 - q0;
  if (n < 0 || pages < 0 || q0 < 0 || p0 < 0 || q1 > tokens) return fail("invalid QIndptr or KvIndptr range");
  int64_t last = last_len[b];
  if (pages > 0 && (last < 1 || last > page_size)) return fail("KvLastPageLength outside [1, BlockSize]");
  int64_t kv_len = pages == 0 ? 0 : (pages - 1) * page_size + last;
  if (kv_len < n && causal) return fail("fewer keys than query tokens");
  if (p1 > kv_indices_len) return fail("KvIndices is shorter than KvIndptr needs");
  s->q0 = q0; s->n = n; s->p0 = p0; s->kv_len = kv_len;
  return 0;
}

int oracle_paged_attention(const void* q, void* out, const void* k_cache, const void* v_cache, int dtype,
                           int kv_dtype, const int32_t* q_indptr, const int32_t* kv_indptr,
                           const int32_t* kv_indices, const int32_t* last_len, int64_t kv_indices_len,
                           int64_t cache_len, int batch, int tokens, int q_heads, int kv_heads, int head_dim,
                           int page_size, int hnd, float scale_arg, float soft_cap, int window_left, int causal,
                           int threads) {
  const int hd = head_dim;
  if (hd < 1 || hd > 1024) return fail("HeadDim must be in [1, 1024]");
  if (kv_heads < 1 || q_heads % kv_heads != 0) return fail("QHeads must be a multiple of KvHeads");
  if (page_size < 1) return fail("BlockSize must be positive");
  if (window_left == 0) return fail("PagedAttention: WindowLeft is 0");
  const double scale = scale_arg == 0.0f ? 1.0 / sqrt((double)hd) : (double)scale_arg;
  const int group = q_heads / kv_heads;
  Seq* seqs = (Seq*)malloc(sizeof(Seq) * (size_t)(batch > 0 ? batch : 1));
  for (int b = 0; b < batch; ++b) {
    /* CpuOps.cs:337-351 CheckAttentionSequence: validate every sequence before the first write. */
    if (attention_sequence(q_indptr, kv_indptr, last_len, kv_indices_len, b, tokens, page_size, causal, &seqs[b])) {
      free(seqs);
      return 1;
    }
    const Seq* s = &seqs[b];
    if (s->n == 0 || s->kv_len == 0) continue;
    int64_t first_key = window_left >= 0 ? (s->kv_len - s->n - window_left > 0 ? s->kv_len - s->n - window_left : 0) : 0;
    for (int64_t page = first_key / page_size; page <= (s->kv_len - 1) / page_size; ++page) {
      if (kv_indices[s->p0 + page] < 0) {
        free(seqs);
        return fail("PagedAttention: a released block is inside a query's window");
      }
    }
  }
  /* Rows are range-checked (NeedRange) before use; a row outside the pool is an error. */
  int err = 0;
  const int64_t work = (int64_t)batch * q_heads;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1) reduction(| : err)
#endif
  for (int64_t bh = 0; bh < work; ++bh) {
    const int b = (int)(bh / q_heads);
    const int h = (int)(bh % q_heads);
    const Seq* s = &seqs[b];
    const int kvh = h / group;
    double* acc = (double*)malloc(sizeof(double) * (size_t)hd);
    for (int64_t i = 0; i < s->n; ++i) {
      const int64_t qpos = s->kv_len - s->n + i;
      const int64_t hi = causal ? qpos : s->kv_len - 1;
      const int64_t lo = window_left >= 0 ? (qpos - window_left > 0 ? qpos - window_left : 0) : 0;
      const int64_t qo = ((s->q0 + i) * q_heads + h) * (int64_t)hd;
      double m = -INFINITY, denom = 0.0;
      for (int d = 0; d < hd; ++d) acc[d] = 0.0;
      for (int64_t j = lo; j <= hi; ++j) {
        const int64_t block = kv_indices[s->p0 + j / page_size];
        const int64_t off = j % page_size;
        const int64_t row = hnd ? ((block * kv_heads + kvh) * page_size + off) * hd
                                : ((block * page_size + off) * kv_heads + kvh) * hd;
        if (row < 0 || row + hd > cache_len) {
          err |= 1;
          break;
        }
        double sc = 0.0;
        for (int d = 0; d < hd; ++d) sc += load(q, dtype, qo + d) * load(k_cache, kv_dtype, row + d);
        sc *= scale;
        if (soft_cap != 0.0f) sc = soft_cap * tanh(sc / soft_cap);
        const double new_m = sc > m ? sc : m;
        const double corr = isinf(m) && m < 0 ? 0.0 : exp(m - new_m);
        const double w = exp(sc - new_m);
        denom = denom * corr + w;
        for (int d = 0; d < hd; ++d) acc[d] = acc[d] * corr + w * load(v_cache, kv_dtype, row + d);
        m = new_m;
      }
      for (int d = 0; d < hd; ++d) store(out, dtype, qo + d, denom == 0.0 ? 0.0 : acc[d] / denom);
    }
    free(acc);
  }
  free(seqs);
  if (err) return fail("a KV row is outside the cache span");
  return 0;
}

/* ---- CacheWrite (reference: src/Starlings.Roost.Ops/CpuOps.cs:515-569; same-dtype byte copy) ---- */

int oracle_cache_write(const void* k, const void* v, void* k_cache, void* v_cache, int dtype,
                       const int64_t* slot_mapping, int64_t cache_len, int tokens, int kv_heads, int head_dim,
                       int page_size, int hnd) {
  const int64_t es = elem_size(dtype);
  const int64_t per_token = (int64_t)kv_heads * head_dim;
  for (int t = 0; t < tokens; ++t) {
    const int64_t slot = slot_mapping[t];
    if (slot < 0) continue;
    const int64_t block = slot / page_size;
    const int64_t off = slot % page_size;
    for (int h = 0; h < kv_heads; ++h) {
      const int64_t dst = hnd ? ((block * kv_heads + h) * page_size + off) * head_dim
                              : ((block * page_size + off) * kv_heads + h) * head_dim;
      if (dst < 0 || dst + head_dim > cache_len) return fail("CacheWrite: slot outside the cache span");
      const int64_t src = t * per_token + (int64_t)h * head_dim;
      memcpy((char*)k_cache + dst * es, (const char*)k + src * es, (size_t)(head_dim * es));
      memcpy((char*)v_cache + dst * es, (const char*)v + src * es, (size_t)(head_dim * es));
    }
  }
  return 0;
}

/* ---- QkNorm and Rope (reference: src/Starlings.Roost.Ops/CpuOps.cs:63-175) ---- */

/* One head row: y = x / sqrt(sum(x^2) / dim + eps) * w, in double, rounded once (CpuOps.cs:89-103). */
static void norm_row(void* x, int dt, int64_t o, const void* w, int dim, float eps) {
  double ss = 0.0;
  for (int i = 0; i < dim; ++i) {
    const double v = load(x, dt, o + i);
    ss += v * v;
  }
  const double inv = 1.0 / sqrt(ss / dim + (double)eps);
  for (int i = 0; i < dim; ++i) store(x, dt, o + i, load(x, dt, o + i) * inv * load(w, dt, i));
}

/* QkNorm (CpuOps.cs:63-87), in place, every query head with q_weight and every key head with k_weight. q_stride and
 * k_stride are the elements between tokens (0: heads * head_dim), as RoostQkNormParams carries them; CpuOps itself
 * has contiguous rows only. */
int oracle_qk_norm(void* q, void* k, const void* q_weight, const void* k_weight, int dtype, int tokens, int q_heads,
                   int kv_heads, int head_dim, int q_stride, int k_stride, float eps) {
  const int64_t qs = q_stride ? q_stride : (int64_t)q_heads * head_dim;
  const int64_t ks = k_stride ? k_stride : (int64_t)kv_heads * head_dim;
  for (int t = 0; t < tokens; ++t) {
    for (int h = 0; h < q_heads; ++h) norm_row(q, dtype, t * qs + (int64_t)h * head_dim, q_weight, head_dim, eps);
  }
  for (int t = 0; t < tokens; ++t) {
    for (int h = 0; h < kv_heads; ++h) norm_row(k, dtype, t * ks + (int64_t)h * head_dim, k_weight, head_dim, eps);
  }
  return 0;
}

/* Frequency i of R rotary dims (CpuOps.cs:141-163): theta^(-2i/R), Llama 3 scaled when kind is 1. */
static double rope_frequency(int i, int rot, double theta, int kind, double factor, double low_ff, double high_ff,
                             double orig) {
  const double f = pow(theta, -2.0 * i / rot);
  if (kind != 1) return f;
  const double wavelen = 2.0 * M_PI / f;
  const double low = orig / low_ff;
  const double high = orig / high_ff;
  if (wavelen < high) return f;
  if (wavelen > low) return f / factor;
  const double smooth = (orig / wavelen - low_ff) / (high_ff - low_ff);
  return (1.0 - smooth) * f / factor + smooth * f;
}

/* Rope (CpuOps.cs:111-175), in place: angle = position * f_i; NeoX pairs (i, i + R/2) or interleaved (2i, 2i + 1)
 * become (x1 cos - x2 sin, x2 cos + x1 sin); elements at and beyond R are unchanged. The float parameters are widened
 * from float as the C# fields are. */
int oracle_rope(void* q, void* k, const int32_t* positions, int dtype, int tokens, int q_heads, int kv_heads,
                int head_dim, int rotary_dim, int kind, int interleaved, float theta, float factor, float low_ff,
                float high_ff, int orig_max) {
  const int rot = rotary_dim == 0 ? head_dim : rotary_dim;
  if (rot < 0 || rot > head_dim || (rot & 1) != 0) return fail("Rope: RotaryDim must be even and at most HeadDim");
  const int half = rot / 2;
  for (int t = 0; t < tokens; ++t) {
    const double pos = positions[t];
    for (int i = 0; i < half; ++i) {
      const double f = rope_frequency(i, rot, theta, kind, factor, low_ff, high_ff, orig_max);
      const double c = cos(pos * f), s = sin(pos * f);
      const int ia = interleaved ? 2 * i : i;
      const int ib = interleaved ? 2 * i + 1 : i + half;
      for (int pass = 0; pass < 2; ++pass) {
        void* x = pass == 0 ? q : k;
        const int heads = pass == 0 ? q_heads : kv_heads;
        for (int h = 0; h < heads; ++h) {
          const int64_t o = ((int64_t)t * heads + h) * head_dim;
          const double x1 = load(x, dtype, o + ia), x2 = load(x, dtype, o + ib);
          store(x, dtype, o + ia, x1 * c - x2 * s);
          store(x, dtype, o + ib, x2 * c + x1 * s);
        }
      }
    }
  }
  return 0;
}

/* ---- GatedDeltaRule (reference: src/Starlings.Roost.Ops/CpuOps.Hybrid.cs:30-157, 233-241) ---- */

/* One (sequence, value head) of GatedDeltaRule: CpuOps' loop body (CpuOps.Hybrid.cs:82-149). */
typedef struct GdnCall {
  const void *q, *k, *v, *g, *beta;
  void* out;
  float* state;
  const int32_t *slots, *cu;
  int g_dtype, beta_dtype, dtype, v_heads, kd, vd, group, use_initial_state, l2_norm_qk;
  int64_t qs, ks, vs, state_elems;
  double scale;
} GdnCall;

static void gdn_unit(const GdnCall* c, int b, int h) {
  const void *q = c->q, *k = c->k, *v = c->v, *g = c->g, *beta = c->beta;
  void* out = c->out;
  const int32_t *slots = c->slots, *cu = c->cu;
  const int g_dtype = c->g_dtype, beta_dtype = c->beta_dtype, dtype = c->dtype, v_heads = c->v_heads;
  const int kd = c->kd, vd = c->vd, group = c->group, use_initial_state = c->use_initial_state;
  const int l2_norm_qk = c->l2_norm_qk;
  const int64_t qs = c->qs, ks = c->ks, vs = c->vs, state_elems = c->state_elems;
  const double scale = c->scale;
  float* state = c->state;
  const int64_t t0 = cu[b], t1 = cu[b + 1];
  if (t1 == t0) return;
  double* s = (double*)malloc(sizeof(double) * (size_t)(state_elems + 2 * kd + vd));
  double* qv = s + state_elems;
  double* kv = qv + kd;
  double* dv = kv + kd;
  float* st = state + ((int64_t)slots[b] * v_heads + h) * state_elems;
  for (int64_t i = 0; i < state_elems; ++i) s[i] = use_initial_state ? (double)st[i] : 0.0;
  const int kh = h / group;
  for (int64_t t = t0; t < t1; ++t) {
    const int64_t qo = t * qs + (int64_t)kh * kd;
    const int64_t ko = t * ks + (int64_t)kh * kd;
    double qq = 0.0, kk = 0.0;
    for (int i = 0; i < kd; ++i) {
      qv[i] = load(q, dtype, qo + i);
      kv[i] = load(k, dtype, ko + i);
      qq += qv[i] * qv[i];
      kk += kv[i] * kv[i];
    }
    const double qn = l2_norm_qk ? 1.0 / sqrt(qq + 1e-6) : 1.0;
    const double kn = l2_norm_qk ? 1.0 / sqrt(kk + 1e-6) : 1.0;
    for (int i = 0; i < kd; ++i) {
      qv[i] *= qn * scale;
      kv[i] *= kn;
    }
    const double decay = exp(load(g, g_dtype, t * v_heads + h));
    const double bt = load(beta, beta_dtype, t * v_heads + h);
    const int64_t vo = t * vs + (int64_t)h * vd;
    const int64_t oo = (t * v_heads + h) * (int64_t)vd;
    for (int j = 0; j < vd; ++j) {
      double kvs = 0.0;
      for (int i = 0; i < kd; ++i) {
        s[(int64_t)i * vd + j] *= decay;
        kvs += s[(int64_t)i * vd + j] * kv[i];
      }
      dv[j] = bt * (load(v, dtype, vo + j) - kvs);
    }
    for (int j = 0; j < vd; ++j) {
      double o = 0.0;
      for (int i = 0; i < kd; ++i) {
        s[(int64_t)i * vd + j] += kv[i] * dv[j];
        o += s[(int64_t)i * vd + j] * qv[i];
      }
      store(out, dtype, oo + j, o);
    }
  }
  for (int64_t i = 0; i < state_elems; ++i) st[i] = (float)s[i];
  free(s);
}

int oracle_gated_delta_rule(const void* q, const void* k, const void* v, const void* g, int g_dtype,
                            const void* beta, int beta_dtype, void* out, float* state, int64_t state_len,
                            const int32_t* slots, const int32_t* cu, int dtype, int batch, int tokens, int k_heads,
                            int v_heads, int k_dim, int v_dim, int64_t q_stride, int64_t k_stride, int64_t v_stride,
                            int use_initial_state, int l2_norm_qk, float scale_arg, int threads) {
  if (k_heads < 1 || v_heads % k_heads != 0) return fail("VHeads must be a multiple of KHeads");
  const int kd = k_dim, vd = v_dim;
  const int64_t qrow = (int64_t)k_heads * kd, vrow = (int64_t)v_heads * vd;
  const int64_t qs = q_stride == 0 ? qrow : q_stride;
  const int64_t ks = k_stride == 0 ? qrow : k_stride;
  const int64_t vs = v_stride == 0 ? vrow : v_stride;
  if (qs < qrow || ks < qrow || vs < vrow) return fail("a stride is smaller than the row width");
  const double scale = scale_arg == 0.0f ? 1.0 / sqrt((double)kd) : (double)scale_arg;
  const int group = v_heads / k_heads;
  const int64_t state_elems = (int64_t)kd * vd;
  for (int b = 0; b < batch; ++b) {
    const int64_t t0 = cu[b], t1 = cu[b + 1];
    if (t0 < 0 || t1 < t0 || t1 > tokens) return fail("invalid CuSeqlens range");
    if (t1 > t0) {
      const int64_t so = ((int64_t)slots[b] * v_heads) * state_elems;
      if (so < 0 || so + (int64_t)v_heads * state_elems > state_len) return fail("state slot outside the pool");
    }
  }
  const GdnCall call = {q, k, v, g, beta, out, state, slots, cu, g_dtype, beta_dtype, dtype, v_heads, kd, vd, group,
                        use_initial_state, l2_norm_qk, qs, ks, vs, state_elems, scale};
  /* CpuOps walks the batch in order, so sequences that share a slot see each other's writes. When any do, the
   * parallel loop runs over heads only, each head walking the batch in order; otherwise over (sequence, head). */
  int shared = 0;
  for (int b = 0; b < batch && !shared; ++b) {
    for (int c2 = b + 1; c2 < batch && !shared; ++c2) {
      shared = slots[b] == slots[c2] && cu[b + 1] > cu[b] && cu[c2 + 1] > cu[c2];
    }
  }
  if (shared) {
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
#endif
    for (int h = 0; h < v_heads; ++h) {
      for (int b = 0; b < batch; ++b) gdn_unit(&call, b, h);
    }
    return 0;
  }
  const int64_t work = (int64_t)batch * v_heads;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
#endif
  for (int64_t bh = 0; bh < work; ++bh) gdn_unit(&call, (int)(bh / v_heads), (int)(bh % v_heads));
  return 0;
}

/* ---- Plan region: slot mapping and batch tables (reference: src/Starlings.Roost.Worker/Eager/PlanRegionWriter.cs:19-64) ---- */

/* Sequences are given as (token_start, token_count, position_offset, kv_length, block list). Writes q_indptr and
 * cu_seqlens [batch+1], kv_indptr [batch+1], kv_indices, kv_last_page_len [batch] and slot_mapping [tokens]. */
int oracle_plan_region(int batch, const int32_t* token_start, const int32_t* token_count,
                       const int32_t* position_offset, const int32_t* kv_length, const int32_t* block_indptr,
                       const int32_t* blocks, int block_size, int32_t* q_indptr, int32_t* cu_seqlens,
                       int32_t* kv_indptr, int32_t* kv_indices, int32_t* kv_last_page_len, int64_t* slot_mapping) {
  int32_t block_at = 0, q_end = 0;
  for (int b = 0; b < batch; ++b) {
    q_indptr[b] = token_start[b];
    cu_seqlens[b] = token_start[b];
    kv_indptr[b] = block_at;
    const int32_t nblocks = block_indptr[b + 1] - block_indptr[b];
    for (int i = 0; i < nblocks; ++i) kv_indices[block_at + i] = blocks[block_indptr[b] + i];
    block_at += nblocks;
    kv_last_page_len[b] = kv_length[b] - (nblocks - 1) * block_size;
    for (int t = 0; t < token_count[b]; ++t) {
      const int32_t index = token_start[b] + t;
      const int32_t position = position_offset[b] + t;
      if (position / block_size >= nblocks) return fail("a position has no block");
      slot_mapping[index] = (int64_t)blocks[block_indptr[b] + position / block_size] * block_size + position % block_size;
    }
    q_end = token_start[b] + token_count[b];
  }
  q_indptr[batch] = q_end;
  cu_seqlens[batch] = q_end;
  kv_indptr[batch] = block_at;
  return 0;
}

/* ---- Gated DeltaNet layer neighbours (reference: src/Starlings.Roost.Ops/CpuOps.Gating.cs:21-110,
 *      CpuOps.Hybrid.cs:160-263, CpuElements.cs:223) ---- */

static double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }
static double silu_d(double x) { return x / (1.0 + exp(-x)); }

/* GatedDeltaRuleGates (CpuOps.Gating.cs:21-47): a and b read as `dtype` at their row strides (0 = v_heads); a_log,
 * dt_bias, g and beta in their own types. softplus(x) = x above 20, else log(1 + exp(x)). */
int oracle_gdn_gates(const void* a, const void* b, int dtype, const void* a_log, int alog_dt, const void* dt_bias,
                     int dtb_dt, void* g, int g_dt, void* beta, int beta_dt, int tokens, int v_heads, int64_t a_stride,
                     int64_t b_stride) {
  const int64_t as = a_stride == 0 ? v_heads : a_stride;
  const int64_t bs = b_stride == 0 ? v_heads : b_stride;
  if (as < v_heads || bs < v_heads) return fail("AStride and BStride must be 0 or at least VHeads");
  for (int64_t t = 0; t < tokens; ++t) {
    for (int h = 0; h < v_heads; ++h) {
      const double x = load(a, dtype, t * as + h) + load(dt_bias, dtb_dt, h);
      const double sp = x > 20.0 ? x : log(1.0 + exp(x));
      store(g, g_dt, t * v_heads + h, -exp(load(a_log, alog_dt, h)) * sp);
      store(beta, beta_dt, t * v_heads + h, sigmoid_d(load(b, dtype, t * bs + h)));
    }
  }
  return 0;
}

/* GatedRmsNorm (CpuOps.Gating.cs:57-86): out = x / sqrt(sum(x^2) / dim + eps) * weight * silu(gate), per row. */
int oracle_gated_rms_norm(const void* x, const void* gate, const void* weight, int w_dt, void* out, int dtype,
                          int64_t rows, int dim, float eps) {
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t o = r * dim;
    double ss = 0.0;
    for (int i = 0; i < dim; ++i) {
      const double v = load(x, dtype, o + i);
      ss += v * v;
    }
    const double inv = 1.0 / sqrt(ss / dim + (double)eps);
    for (int i = 0; i < dim; ++i) {
      const double y = load(x, dtype, o + i) * inv * load(weight, w_dt, i) * silu_d(load(gate, dtype, o + i));
      store(out, dtype, o + i, y);
    }
  }
  return 0;
}

/* SigmoidMul (CpuOps.Gating.cs:91-101): out = x / (1 + exp(-gate)) elementwise. */
int oracle_sigmoid_mul(const void* x, const void* gate, void* out, int dtype, int64_t n) {
  for (int64_t i = 0; i < n; ++i) store(out, dtype, i, load(x, dtype, i) * sigmoid_d(load(gate, dtype, i)));
  return 0;
}

/* CausalConv1d (CpuOps.Hybrid.cs:167-243): y_t = bias + sum_j weight[c, j] * h_{t + j}, h = [state (width - 1, oldest
 * first), inputs]; silu last when set; then the slot holds the last width - 1 entries of h. Weight and bias are read
 * as `dtype`, the state as `state_dt`. A sequence of zero tokens leaves its slot untouched. */
int oracle_causal_conv1d(const void* x, const void* weight, const void* bias, void* out, int dtype, void* state,
                         int state_dt, int64_t state_len, const int32_t* slots, const int32_t* cu, int batch, int tokens,
                         int channels, int width, int silu) {
  if (width < 1 || width > 16) return fail("Width must be in [1, 16]");
  const int sl = width - 1;
  double next[16];
  for (int b = 0; b < batch; ++b) {
    const int64_t t0 = cu[b], t1 = cu[b + 1];
    if (t0 < 0 || t1 < t0 || t1 > tokens) return fail("invalid CuSeqlens range");
    const int64_t n = t1 - t0;
    if (n == 0) continue;
    for (int c = 0; c < channels; ++c) {
      const int64_t so = ((int64_t)slots[b] * channels + c) * sl;
      if (so < 0 || so + sl > state_len) return fail("conv state slot outside the pool");
#define HIST(i) ((i) < sl ? load(state, state_dt, so + (i)) : load(x, dtype, (t0 + (i) - sl) * channels + c))
      for (int64_t t = 0; t < n; ++t) {
        double y = bias != NULL ? load(bias, dtype, c) : 0.0;
        for (int j = 0; j < width; ++j) y += load(weight, dtype, (int64_t)c * width + j) * HIST(t + j);
        store(out, dtype, (t0 + t) * channels + c, silu ? silu_d(y) : y);
      }
      for (int j = 0; j < sl; ++j) next[j] = HIST(n + j);
#undef HIST
      for (int j = 0; j < sl; ++j) store(state, state_dt, so + j, next[j]);
    }
  }
  return 0;
}

/* RecurrentStateCopy / RecurrentStateSnapshot (CpuOps.Hybrid.cs:251-263): byte copies of slot_bytes, pair by pair in
 * order. copy: src = dst = pool, pairs (from, to); snapshot: pairs (slot, snapshot), restore swaps the direction. */
int oracle_state_copy_pairs(const uint8_t* src, int64_t src_bytes, uint8_t* dst, int64_t dst_bytes,
                            const int32_t* pairs, int count, int64_t slot_bytes, int swap) {
  for (int i = 0; i < count; ++i) {
    const int64_t from = (int64_t)pairs[2 * i + swap], to = (int64_t)pairs[2 * i + 1 - swap];
    if (from < 0 || to < 0 || (from + 1) * slot_bytes > src_bytes || (to + 1) * slot_bytes > dst_bytes) {
      return fail("a slot lies outside its pool");
    }
    memmove(dst + to * slot_bytes, src + from * slot_bytes, (size_t)slot_bytes);
  }
  return 0;
}
