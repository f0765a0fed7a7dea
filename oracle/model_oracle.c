/*
 * CPU oracle for the decode step around the Linear path — TEST
 * INFRASTRUCTURE ONLY (see model_oracle.h for what it restates and how each
 * function is pinned).  Built with -ffp-contract=off like linear_oracle.c.
 */
#include "model_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#include "linear_oracle.h"

/* cpu_ops.cpp:15-21. */
void orc_rms_norm(const float* input, const float* weight, float* output, int n,
                  float epsilon) {
  double sum = 0.0;
  for (int i = 0; i < n; ++i) sum += (double)input[i] * input[i];
  const float scale = 1.0f / sqrtf((float)(sum / n) + epsilon);
  for (int i = 0; i < n; ++i) output[i] = input[i] * scale * weight[i];
}

static void rope_heads(float* data, int heads, int head_dim, int position, float theta) {
  const int half = head_dim / 2;
  for (int head = 0; head < heads; ++head) {
    float* values = data + (size_t)head * head_dim;
    for (int i = 0; i < half; ++i) {
      const float frequency = powf(theta, -2.0f * (float)i / (float)head_dim);
      const float angle = (float)position * frequency;
      const float cosine = cosf(angle);
      const float sine = sinf(angle);
      const float first = values[i];
      const float second = values[i + half];
      values[i] = first * cosine - second * sine;
      values[i + half] = second * cosine + first * sine;
    }
  }
}

/* cpu_ops.cpp:33-56. */
void orc_rope(float* q, float* k, int num_heads, int num_kv_heads, int head_dim,
              int position, float theta) {
  rope_heads(q, num_heads, head_dim, position, theta);
  rope_heads(k, num_kv_heads, head_dim, position, theta);
}

/* cpu_ops.cpp:58-91, one head. */
static void attention_head(const float* query, const float* key_cache,
                           const float* value_cache, float* head_output, int head_dim,
                           int sequence_length, float* scores) {
  const float scale = 1.0f / sqrtf((float)head_dim);
  float maximum = -INFINITY;
  for (int pos = 0; pos < sequence_length; ++pos) {
    const float* key = key_cache + (size_t)pos * head_dim;
    float dot = 0.0f;
    for (int d = 0; d < head_dim; ++d) dot += query[d] * key[d];
    scores[pos] = dot * scale;
    if (scores[pos] > maximum) maximum = scores[pos];
  }
  float denominator = 0.0f;
  for (int pos = 0; pos < sequence_length; ++pos) {
    scores[pos] = expf(scores[pos] - maximum);
    denominator += scores[pos];
  }
  for (int d = 0; d < head_dim; ++d) head_output[d] = 0.0f;
  for (int pos = 0; pos < sequence_length; ++pos) {
    const float probability = scores[pos] / denominator;
    const float* value = value_cache + (size_t)pos * head_dim;
    for (int d = 0; d < head_dim; ++d) head_output[d] += probability * value[d];
  }
}

void orc_attention_decode(const float* q, const float* key_cache,
                          const float* value_cache, float* output, int num_heads,
                          int num_kv_heads, int head_dim, int sequence_length,
                          int max_sequence_length, int threads) {
  const int heads_per_kv = num_heads / num_kv_heads;
  const int nt = threads > 0 ? threads : orc_default_threads();
#pragma omp parallel num_threads(nt)
  {
    float* scores = (float*)malloc((size_t)(sequence_length > 0 ? sequence_length : 1) *
                                   sizeof(float));
#pragma omp for schedule(static)
    for (int head = 0; head < num_heads; ++head) {
      const int kv_head = head / heads_per_kv;
      const size_t base = (size_t)kv_head * max_sequence_length * head_dim;
      attention_head(q + (size_t)head * head_dim, key_cache + base, value_cache + base,
                     output + (size_t)head * head_dim, head_dim, sequence_length, scores);
    }
    free(scores);
  }
}

/* cpu_ops.cpp:168-173. */
void orc_silu_mul(const float* gate, const float* up, float* output, int n) {
  for (int i = 0; i < n; ++i) {
    const float silu = gate[i] / (1.0f + expf(-gate[i]));
    output[i] = silu * up[i];
  }
}

struct orc_model {
  orc_model_config c;
  orc_model_weights w;
  int head_dim;
  int kv_dim;
  float* key_cache;    /* [layers][kv_heads][max_seq][head_dim] */
  float* value_cache;  /* same */
  /* one token's activations */
  float *x, *norm, *q, *k, *v, *attn, *tmp, *gate, *up, *mlp, *logits;
};

orc_model* orc_model_create(const orc_model_config* config,
                            const orc_model_weights* weights) {
  if (!config || !weights || config->layers <= 0 || config->hidden <= 0 ||
      config->heads <= 0 || config->kv_heads <= 0 || config->heads % config->kv_heads ||
      config->hidden % config->heads || config->inter <= 0 || config->vocab <= 0 ||
      config->max_seq <= 0) {
    return NULL;
  }
  orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
  if (!m) return NULL;
  m->c = *config;
  m->w = *weights;
  m->head_dim = config->hidden / config->heads;
  m->kv_dim = config->kv_heads * m->head_dim;
  const size_t cache = (size_t)config->layers * config->kv_heads * config->max_seq * m->head_dim;
  m->key_cache = (float*)calloc(cache, sizeof(float));
  m->value_cache = (float*)calloc(cache, sizeof(float));
  const int h = config->hidden, i = config->inter;
  m->x = (float*)malloc(sizeof(float) * (size_t)(6 * h + 2 * m->kv_dim + 3 * i + config->vocab));
  if (!m->key_cache || !m->value_cache || !m->x) {
    orc_model_destroy(m);
    return NULL;
  }
  m->norm = m->x + h;
  m->q = m->norm + h;
  m->attn = m->q + h;
  m->tmp = m->attn + h;
  m->k = m->tmp + h;
  m->v = m->k + m->kv_dim;
  m->gate = m->v + m->kv_dim;
  m->up = m->gate + i;
  m->mlp = m->up + i;
  m->logits = m->mlp + i;
  return m;
}

void orc_model_destroy(orc_model* m) {
  if (!m) return;
  free(m->key_cache);
  free(m->value_cache);
  free(m->x);
  free(m);
}

static const float* layer_bias(const float* base, int layer, int size) {
  return base ? base + (size_t)layer * size : NULL;
}

static float* cache_of(orc_model* m, float* cache, int layer) {
  return cache + (size_t)layer * m->c.kv_heads * m->c.max_seq * m->head_dim;
}

/* qwen2.cpp:376-425. */
int orc_model_decode(orc_model* m, int token, int position, float* logits) {
  if (!m) return -1;
  const orc_model_config* c = &m->c;
  const orc_model_weights* w = &m->w;
  const int h = c->hidden, kv = m->kv_dim, hd = m->head_dim, in = c->inter, nt = c->threads;
  if (token < 0 || token >= c->vocab || position < 0 || position >= c->max_seq) return -1;
  memcpy(m->x, w->embed + (size_t)token * h, sizeof(float) * h);
  for (int l = 0; l < c->layers; ++l) {
    orc_rms_norm(m->x, w->in_norm + (size_t)l * h, m->norm, h, c->eps);
    orc_linear_fp32(w->wq + (size_t)l * h * h, layer_bias(w->bq, l, h), m->norm, m->q, h, h, nt);
    orc_linear_fp32(w->wk + (size_t)l * kv * h, layer_bias(w->bk, l, kv), m->norm, m->k, kv, h,
                    nt);
    orc_linear_fp32(w->wv + (size_t)l * kv * h, layer_bias(w->bv, l, kv), m->norm, m->v, kv, h,
                    nt);
    orc_rope(m->q, m->k, c->heads, c->kv_heads, hd, position, c->theta);
    float* kc = cache_of(m, m->key_cache, l);
    float* vc = cache_of(m, m->value_cache, l);
    for (int head = 0; head < c->kv_heads; ++head) {
      const size_t at = ((size_t)head * c->max_seq + position) * hd;
      memcpy(kc + at, m->k + head * hd, sizeof(float) * hd);
      memcpy(vc + at, m->v + head * hd, sizeof(float) * hd);
    }
    orc_attention_decode(m->q, kc, vc, m->attn, c->heads, c->kv_heads, hd, position + 1,
                         c->max_seq, nt);
    orc_linear_fp32(w->wo + (size_t)l * h * h, NULL, m->attn, m->tmp, h, h, nt);
    for (int i = 0; i < h; ++i) m->x[i] += m->tmp[i];
    orc_rms_norm(m->x, w->post_norm + (size_t)l * h, m->norm, h, c->eps);
    orc_linear_fp32(w->wg + (size_t)l * in * h, NULL, m->norm, m->gate, in, h, nt);
    orc_linear_fp32(w->wu + (size_t)l * in * h, NULL, m->norm, m->up, in, h, nt);
    orc_silu_mul(m->gate, m->up, m->mlp, in);
    orc_linear_fp32(w->wd + (size_t)l * h * in, NULL, m->mlp, m->tmp, h, in, nt);
    for (int i = 0; i < h; ++i) m->x[i] += m->tmp[i];
  }
  orc_rms_norm(m->x, w->final_norm, m->norm, h, c->eps);
  orc_linear_fp32(w->embed, NULL, m->norm, m->logits, c->vocab, h, nt);
  if (logits) memcpy(logits, m->logits, sizeof(float) * c->vocab);
  return orc_argmax(m->logits, c->vocab);
}

/* qwen2.cpp:427-494. */
int orc_model_prefill(orc_model* m, const int* tokens, int count, float* logits) {
  if (!m) return -1;
  const orc_model_config* c = &m->c;
  const orc_model_weights* w = &m->w;
  const int h = c->hidden, kv = m->kv_dim, hd = m->head_dim, in = c->inter, nt = c->threads;
  if (!tokens || count <= 0 || count > c->max_seq) return -1;
  for (int t = 0; t < count; ++t) {
    if (tokens[t] < 0 || tokens[t] >= c->vocab) return -1;
  }
  const size_t n = (size_t)count;
  float* buf = (float*)malloc(sizeof(float) * n * (5 * (size_t)h + 2 * (size_t)kv + 3 * (size_t)in));
  if (!buf) return -1;
  float *x = buf, *norm = x + n * h, *q = norm + n * h, *attn = q + n * h, *tmp = attn + n * h;
  float *k = tmp + n * h, *v = k + n * kv, *gate = v + n * kv, *up = gate + n * in,
        *mlp = up + n * in;
  for (int t = 0; t < count; ++t) {
    memcpy(x + (size_t)t * h, w->embed + (size_t)tokens[t] * h, sizeof(float) * h);
  }
  for (int l = 0; l < c->layers; ++l) {
    for (int t = 0; t < count; ++t) {
      orc_rms_norm(x + (size_t)t * h, w->in_norm + (size_t)l * h, norm + (size_t)t * h, h,
                   c->eps);
    }
    orc_linear_fp32_batch(w->wq + (size_t)l * h * h, layer_bias(w->bq, l, h), norm, q, count,
                          h, h, nt);
    orc_linear_fp32_batch(w->wk + (size_t)l * kv * h, layer_bias(w->bk, l, kv), norm, k,
                          count, kv, h, nt);
    orc_linear_fp32_batch(w->wv + (size_t)l * kv * h, layer_bias(w->bv, l, kv), norm, v,
                          count, kv, h, nt);
    for (int t = 0; t < count; ++t) {
      orc_rope(q + (size_t)t * h, k + (size_t)t * kv, c->heads, c->kv_heads, hd, t, c->theta);
    }
    float* kc = cache_of(m, m->key_cache, l);
    float* vc = cache_of(m, m->value_cache, l);
    for (int t = 0; t < count; ++t) {
      for (int head = 0; head < c->kv_heads; ++head) {
        const size_t at = ((size_t)head * c->max_seq + t) * hd;
        memcpy(kc + at, k + (size_t)t * kv + head * hd, sizeof(float) * hd);
        memcpy(vc + at, v + (size_t)t * kv + head * hd, sizeof(float) * hd);
      }
    }
    for (int t = 0; t < count; ++t) {
      orc_attention_decode(q + (size_t)t * h, kc, vc, attn + (size_t)t * h, c->heads,
                           c->kv_heads, hd, t + 1, c->max_seq, nt);
    }
    orc_linear_fp32_batch(w->wo + (size_t)l * h * h, NULL, attn, tmp, count, h, h, nt);
    for (size_t i = 0; i < n * h; ++i) x[i] += tmp[i];
    for (int t = 0; t < count; ++t) {
      orc_rms_norm(x + (size_t)t * h, w->post_norm + (size_t)l * h, norm + (size_t)t * h, h,
                   c->eps);
    }
    orc_linear_fp32_batch(w->wg + (size_t)l * in * h, NULL, norm, gate, count, in, h, nt);
    orc_linear_fp32_batch(w->wu + (size_t)l * in * h, NULL, norm, up, count, in, h, nt);
    orc_silu_mul(gate, up, mlp, (int)(n * in));
    orc_linear_fp32_batch(w->wd + (size_t)l * h * in, NULL, mlp, tmp, count, h, in, nt);
    for (size_t i = 0; i < n * h; ++i) x[i] += tmp[i];
  }
  orc_rms_norm(x + (size_t)(count - 1) * h, w->final_norm, m->norm, h, c->eps);
  orc_linear_fp32(w->embed, NULL, m->norm, m->logits, c->vocab, h, nt);
  free(buf);
  if (logits) memcpy(logits, m->logits, sizeof(float) * c->vocab);
  return orc_argmax(m->logits, c->vocab);
}
