/* sampler.c - TEST INFRASTRUCTURE ONLY (see oracle.h).
 * TInferSampler restated from src/infer/mormot.ai.infer.sampler.pas: the
 * warpers of Hugging Face's generate() in its order (temperature, top-k with
 * the ties of the k-th logit, top-p over what top-k kept, min-p), one draw from
 * a splitmix64 stream seeded per sampler (the published generator of Vigna).
 * The candidate threshold is lowered as the reference does, the candidates are
 * ordered by (logit descending, id ascending): a total order, so any correct
 * sort gives the reference's heap-sort order. */
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include "oracle.h"

typedef struct {
  double temperature, top_p, min_p;
  int32_t top_k;
  uint64_t state;
  double* probs;
  int32_t* cand;
  int64_t cap;
} orc_sampler;

static int nonfinite_d(double v)
{
  uint64_t b;
  memcpy(&b, &v, 8);
  return (b & 0x7ff0000000000000ull) == 0x7ff0000000000000ull;
}

static uint32_t fbits(float f)
{
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}

/* sampler.pas:225-238 (splitmix64, 53 bits in [0, 1)) */
double orc_splitmix_next(uint64_t* state)
{
  *state += 0x9E3779B97F4A7C15ull;
  uint64_t z = *state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z = z ^ (z >> 31);
  return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

/* sampler.pas:210-223: NaN, infinities and settings out of range refused */
int orc_sampler_create(double temperature, int32_t top_k, double top_p, double min_p,
                       int64_t seed, void** out)
{
  *out = NULL;
  if (nonfinite_d(temperature) || nonfinite_d(top_p) || nonfinite_d(min_p) || top_k < 0 ||
      top_p <= 0 || top_p > 1 || min_p < 0 || min_p >= 1)
    return -1;
  orc_sampler* s = calloc(1, sizeof *s);
  if (!s) return -6;
  s->temperature = temperature;
  s->top_k = top_k;
  s->top_p = top_p;
  s->min_p = min_p;
  s->state = (uint64_t)seed;
  *out = s;
  return 0;
}

void orc_sampler_destroy(void* h)
{
  orc_sampler* s = h;
  if (!s) return;
  free(s->probs);
  free(s->cand);
  free(s);
}

static const float* g_logits; /* the running Next: the order of qsort */

/* sampler.pas:244-249: the higher logit first, the lower id on a tie */
static int before(const void* pa, const void* pb)
{
  int32_t a = *(const int32_t*)pa, b = *(const int32_t*)pb;
  float la = g_logits[a], lb = g_logits[b];
  if (la > lb) return -1;
  if (lb > la) return 1;
  return a < b ? -1 : (a > b);
}

/* sampler.pas:269-435 */
int64_t orc_sampler_next(void* h, const float* logits, int64_t count)
{
  orc_sampler* s = h;
  if (s->temperature <= 0) return orc_argmax(logits, count);
  if (s->cap < count) {
    free(s->probs);
    free(s->cand);
    s->probs = malloc((size_t)count * sizeof(double));
    s->cand = malloc((size_t)count * sizeof(int32_t));
    s->cap = count;
  }
  double* p = s->probs;
  int32_t* cand = s->cand;
  const int64_t best = orc_argmax(logits, count);
  const double m = logits[best];
  const uint32_t bb = fbits(logits[best]);
  if (((bb & 0x7f800000u) == 0x7f800000u && (bb & 0x007fffffu)) || (bb & 0x7fffffffu) == 0x7f800000u)
    return best; /* no finite best */
  if (s->temperature < 1e-30) return best;
  const double inv = 1.0 / s->temperature;
  double sum = 0;
  for (int64_t i = 0; i < count; i++) {
    if ((fbits(logits[i]) & 0x7f800000u) == 0x7f800000u) p[i] = 0;
    else p[i] = exp(((double)logits[i] - m) * inv);
    sum = sum + p[i];
  }
  for (int64_t i = 0; i < count; i++) p[i] = p[i] / sum;
  if (s->top_k == 0 && s->top_p >= 1 && s->min_p == 0) {
    const double u = orc_splitmix_next(&s->state);
    double cum = 0;
    for (int64_t i = 0; i < count; i++) {
      cum = cum + p[i];
      if (p[i] > 0 && u < cum) return i;
    }
    return best;
  }
  double t = (s->top_k > 0 || s->top_p < 1) ? p[best] * 1e-3 : p[best] * s->min_p;
  int64_t n;
  for (;;) {
    double above = 0;
    n = 0;
    for (int64_t i = 0; i < count; i++)
      if (p[i] >= t && (fbits(logits[i]) & 0x7f800000u) != 0x7f800000u) {
        cand[n++] = (int32_t)i;
        above = above + p[i];
      }
    int enough = s->top_k > 0 ? n >= s->top_k : (s->top_p < 1 ? above >= s->top_p : 1);
    if (enough || t == 0) break;
    t = t * 1e-3;
    if (t < 1e-300) t = 0;
  }
  g_logits = logits;
  qsort(cand, (size_t)n, sizeof(int32_t), before);
  if (s->top_k > 0 && n > s->top_k) {
    int64_t keep = s->top_k;
    while (keep < n && logits[cand[keep]] == logits[cand[s->top_k - 1]]) keep++;
    n = keep;
  }
  if (s->top_p < 1) {
    double mass = 1;
    if (s->top_k > 0) {
      mass = 0;
      for (int64_t i = 0; i < n; i++) mass = mass + p[cand[i]];
    }
    double cum = 0;
    int64_t keep = n;
    for (int64_t i = 0; i < n; i++) {
      cum = cum + p[cand[i]];
      if (cum >= s->top_p * mass) {
        keep = i + 1;
        break;
      }
    }
    n = keep;
  }
  if (s->min_p > 0) {
    int64_t keep = 1;
    while (keep < n && p[cand[keep]] >= s->min_p * p[cand[0]]) keep++;
    n = keep;
  }
  double tot = 0;
  for (int64_t i = 0; i < n; i++) tot = tot + p[cand[i]];
  const double u = orc_splitmix_next(&s->state) * tot;
  double cum = 0;
  for (int64_t i = 0; i < n; i++) {
    cum = cum + p[cand[i]];
    if (u < cum) return cand[i];
  }
  return cand[0];
}
