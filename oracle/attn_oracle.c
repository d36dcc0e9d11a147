/*
 * CPU oracle (test infrastructure only) for the paged attention path.
 *
 * A plain-C restatement of yaxus-backend-cpu's arithmetic on this path:
 *   - dot            crates/yaxus-backend-cpu/src/lib.rs:280-294 (16 lanes, then the rest)
 *   - rmsnorm_row    crates/yaxus-backend-cpu/src/lib.rs:296-302
 *   - rope_inplace   crates/yaxus-backend-cpu/src/lib.rs:304-311
 *   - Rope::cos_sin  crates/yaxus-model/src/config.rs:213-219
 *   - write_rows     crates/yaxus-backend-cpu/src/lib.rs:359-385
 *   - attend         crates/yaxus-backend-cpu/src/lib.rs:389-427 (two-pass softmax)
 *   - copy_page      crates/yaxus-backend-cpu/src/lib.rs:472-479
 *   - matmul (bf16)  crates/yaxus-backend-cpu/src/lib.rs:234-248, 314-345 (dot_bf16)
 *   - argmax         crates/yaxus-backend-cpu/src/lib.rs:432-440
 * The KV arena has the reference's layout, slot-major `[slot][hkv * d]` per layer
 * (lib.rs:205-214), stored as f32 or, in f16 mode, as IEEE binary16 bits rounded to
 * nearest-even from f32 (the `half` 2.7.1 crate's rounding). Arithmetic is f32
 * throughout; build with -ffp-contract=off so no multiply-add is fused.
 *
 * It is the checker for the HIP kernels and the CPU baseline of bench.py; the shipped
 * library never links or calls it. Pinned by: the reference test
 * `paged_attention_matches_dense_attention` (lib.rs:676-714, restated with its xorshift
 * values), an f64 brute-force dense attention, invariants (one key gives V, equal
 * scores give the mean of V, page-permutation invariance) and, for the f16 rounding,
 * an exhaustive comparison with numpy's IEEE conversion over every f16 boundary.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- binary16 <-> binary32 ------------------------------------------------------ */

/* Round-to-nearest-even f32 -> f16 bits, subnormals kept, overflow to infinity, NaN
 * kept as a quiet NaN with the top mantissa bits. */
uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) {
    if (man == 0) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | (man >> 13));
  }
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    /* Subnormal (or zero) result: value = man24 * 2^(exp-150); f16 unit 2^-24. */
    if (e < -10) return (uint16_t)sign; /* below half the smallest subnormal */
    uint32_t m = man | 0x800000u;       /* 24-bit significand */
    uint32_t shift = (uint32_t)(14 - e); /* bits dropped: 13 + (1 - e) */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1;
    return (uint16_t)(sign | q);
  }
  uint32_t q = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1; /* may carry into exp */
  return (uint16_t)(sign | q);
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t x;
  if (exp == 0) {
    if (man == 0) {
      x = sign;
    } else {
      int e = -1;
      do {
        man <<= 1;
        e++;
      } while (!(man & 0x400u));
      x = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    x = sign | 0x7f800000u | (man << 13);
  } else {
    x = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

void orc_f32_to_f16_n(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16(in[i]);
}

static float g_f16_table[65536];
static int g_f16_table_ready = 0;
static pthread_once_t g_once = PTHREAD_ONCE_INIT;
static void build_table(void) {
  for (uint32_t i = 0; i < 65536; ++i) g_f16_table[i] = orc_f16_to_f32((uint16_t)i);
  g_f16_table_ready = 1;
}

/* ---- the CPU backend's primitives ---------------------------------------------- */

/* lib.rs:280-294: 16 accumulators over whole chunks, summed in order, then the rest. */
float orc_dot(const float* a, const float* b, size_t n) {
  float acc[16] = {0};
  size_t chunks = n / 16;
  for (size_t c = 0; c < chunks; ++c)
    for (int i = 0; i < 16; ++i) acc[i] += a[c * 16 + i] * b[c * 16 + i];
  float s = 0.0f;
  for (int i = 0; i < 16; ++i) s += acc[i];
  for (size_t i = chunks * 16; i < n; ++i) s += a[i] * b[i];
  return s;
}

/* lib.rs:109-111 (yaxus-model weights.rs): bf16 is the upper half of an f32. */
static inline float bf16_to_f32(uint16_t b) {
  union { uint32_t u; float f; } v;
  v.u = (uint32_t)b << 16;
  return v.f;
}

/* lib.rs:234-248 (dot_bf16) inside lib.rs:314-345 (matmul): out[i][j] = w[j] . x[i] with
 * 16 accumulators over whole chunks of 16, summed in order, then the rest. (For four or
 * more rows the CPU decodes the row to f32 first and calls dot (lib.rs:280-294): the same
 * products in the same order, so the same bits.) */
void orc_matmul_bf16(const float* x, size_t t, size_t k, const uint16_t* w, size_t n, float* out) {
  for (size_t j = 0; j < n; ++j) {
    const uint16_t* wr = w + j * k;
    for (size_t i = 0; i < t; ++i) {
      const float* xr = x + i * k;
      float acc[16] = {0};
      const size_t chunks = k / 16;
      for (size_t c = 0; c < chunks; ++c)
        for (int l = 0; l < 16; ++l) acc[l] += bf16_to_f32(wr[c * 16 + l]) * xr[c * 16 + l];
      float s = 0.0f;
      for (int l = 0; l < 16; ++l) s += acc[l];
      for (size_t e = chunks * 16; e < k; ++e) s += bf16_to_f32(wr[e]) * xr[e];
      out[i * n + j] = s;
    }
  }
}

/* lib.rs:432-440: the first index whose value is strictly larger than every earlier one,
 * starting from (0, -inf): NaN never wins, a row of -inf / NaN gives 0. */
uint32_t orc_argmax(const float* row, size_t n) {
  size_t best = 0;
  float best_v = -INFINITY;
  for (size_t i = 0; i < n; ++i)
    if (row[i] > best_v) {
      best = i;
      best_v = row[i];
    }
  return (uint32_t)best;
}

/* lib.rs:296-302 */
void orc_rmsnorm_row(const float* x, const float* w, float offset, float eps, float* out,
                     size_t n) {
  float ss = 0.0f;
  for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];
  float ms = ss / (float)n;
  float r = 1.0f / sqrtf(ms + eps);
  for (size_t i = 0; i < n; ++i) out[i] = (offset + w[i]) * (x[i] * r);
}

/* lib.rs:304-311 */
void orc_rope_inplace(float* x, const float* cs, const float* sn, size_t n) {
  size_t half = n / 2;
  for (size_t j = 0; j < half; ++j) {
    float a = x[j], b = x[j + half];
    x[j] = a * cs[j] - b * sn[j];
    x[j + half] = b * cs[j] + a * sn[j];
  }
}

/* config.rs:213-219: the angle in f32 (torch's f32 einsum), cos/sin in f64. */
void orc_cos_sin(const float* inv_freq, size_t half, float concentration, size_t pos,
                 float* cs, float* sn) {
  for (size_t j = 0; j < half; ++j) {
    float a = (float)pos * inv_freq[j];
    cs[j] = (float)cos((double)a) * concentration;
    sn[j] = (float)sin((double)a) * concentration;
  }
}

/* ---- the arena -------------------------------------------------------------------- */

typedef struct {
  size_t slots, kvd;
  int f16;
  void* k;
  void* v;
} orc_layer;

static inline float kv_get(const void* base, int f16, size_t idx) {
  return f16 ? g_f16_table[((const uint16_t*)base)[idx]] : ((const float*)base)[idx];
}
static inline void kv_put(void* base, int f16, size_t idx, float x) {
  if (f16)
    ((uint16_t*)base)[idx] = orc_f32_to_f16(x);
  else
    ((float*)base)[idx] = x;
}

/* Stores raw K/V rows ([rows][hkv*d] each) at their slots: the store half of
 * write_rows (lib.rs:378-383) for inputs that are already normalised and rotated. */
void orc_store_kv(void* kc, void* vc, int f16, size_t kvd, size_t rows, const uint32_t* kv_slot,
                  const float* k, const float* v) {
  pthread_once(&g_once, build_table);
  for (size_t i = 0; i < rows; ++i)
    for (size_t j = 0; j < kvd; ++j) {
      size_t idx = (size_t)kv_slot[i] * kvd + j;
      kv_put(kc, f16, idx, k[i * kvd + j]);
      kv_put(vc, f16, idx, v[i * kvd + j]);
    }
}

/* lib.rs:359-385: per row, q heads normed + rotated to `q`; k normed + rotated and v
 * raw, stored at the row's slot. `qkv` is [rows][(hq + 2 hkv) d]; cos/sin per row
 * from (inv_freq, concentration) at pos[i]. */
void orc_write_rows(const float* qkv, size_t rows, size_t hq, size_t hkv, size_t d,
                    const float* qn, const float* kn, float eps, const float* inv_freq,
                    float concentration, const uint32_t* pos, const uint32_t* kv_slot, void* kc,
                    void* vc, int f16, float* q) {
  pthread_once(&g_once, build_table);
  size_t qd = hq * d, kvd = hkv * d, cols = qd + 2 * kvd;
  float* cs = (float*)malloc(sizeof(float) * d / 2);
  float* sn = (float*)malloc(sizeof(float) * d / 2);
  float* tmp = (float*)malloc(sizeof(float) * d);
  for (size_t i = 0; i < rows; ++i) {
    const float* row = qkv + i * cols;
    orc_cos_sin(inv_freq, d / 2, concentration, pos[i], cs, sn);
    for (size_t h = 0; h < hq; ++h) {
      float* dst = q + i * qd + h * d;
      orc_rmsnorm_row(row + h * d, qn, 1.0f, eps, dst, d);
      orc_rope_inplace(dst, cs, sn, d);
    }
    size_t slot = kv_slot[i];
    for (size_t h = 0; h < hkv; ++h) {
      orc_rmsnorm_row(row + qd + h * d, kn, 1.0f, eps, tmp, d);
      orc_rope_inplace(tmp, cs, sn, d);
      for (size_t j = 0; j < d; ++j) {
        kv_put(kc, f16, slot * kvd + h * d + j, tmp[j]);
        kv_put(vc, f16, slot * kvd + h * d + j, row[qd + kvd + h * d + j]);
      }
    }
  }
  free(cs);
  free(sn);
  free(tmp);
}

/* lib.rs:472-479 */
void orc_copy_page(void* kc, void* vc, int f16, size_t kvd, size_t page, uint32_t src,
                   uint32_t dst) {
  size_t n = page * kvd, es = f16 ? 2 : 4;
  memmove((char*)kc + (size_t)dst * n * es, (char*)kc + (size_t)src * n * es, n * es);
  memmove((char*)vc + (size_t)dst * n * es, (char*)vc + (size_t)src * n * es, n * es);
}

/* ---- attend ------------------------------------------------------------------------ */

typedef struct {
  const float* q;
  size_t rows, hq, hkv, d, page, window;
  const uint32_t* pos;
  const uint32_t* pt_off;
  const uint32_t* pages;
  const void* kc;
  const void* vc;
  int f16;
  float* out;
  size_t u0, u1; /* (row, head) units [u0, u1) */
} attend_job;

/* lib.rs:389-427 for the units of one job. */
static void attend_units(const attend_job* j) {
  size_t hq = j->hq, d = j->d, qd = hq * d, kvd = j->hkv * d, group = hq / j->hkv;
  float scale = 1.0f / sqrtf((float)d);
  float* kbuf = (float*)malloc(sizeof(float) * d);
  size_t cap = 0;
  float* scores = NULL;
  for (size_t idx = j->u0; idx < j->u1; ++idx) {
    size_t i = idx / hq, h = idx % hq, kh = h / group;
    size_t p = j->pos[i];
    size_t lo = 0;
    if (j->window) lo = (p + 1 > j->window) ? p + 1 - j->window : 0;
    size_t n = p + 1 - lo;
    if (n > cap) {
      cap = n;
      scores = (float*)realloc(scores, sizeof(float) * cap);
    }
    const float* qv = j->q + i * qd + h * d;
    const uint32_t* pt = j->pages + j->pt_off[i];
    for (size_t s = lo; s <= p; ++s) {
      size_t slot = (size_t)pt[s / j->page] * j->page + s % j->page;
      size_t off = slot * kvd + kh * d;
      for (size_t e = 0; e < d; ++e) kbuf[e] = kv_get(j->kc, j->f16, off + e);
      scores[s - lo] = orc_dot(qv, kbuf, d) * scale;
    }
    float m = -INFINITY;
    for (size_t s = 0; s < n; ++s) m = fmaxf(m, scores[s]);
    float* o = j->out + i * qd + h * d;
    for (size_t e = 0; e < d; ++e) o[e] = 0.0f;
    float denom = 0.0f;
    for (size_t s = lo; s <= p; ++s) {
      float ex = expf(scores[s - lo] - m);
      denom += ex;
      size_t slot = (size_t)pt[s / j->page] * j->page + s % j->page;
      size_t off = slot * kvd + kh * d;
      for (size_t e = 0; e < d; ++e) o[e] += ex * kv_get(j->vc, j->f16, off + e);
    }
    for (size_t e = 0; e < d; ++e) o[e] /= denom;
  }
  free(kbuf);
  free(scores);
}

static void* attend_thread(void* arg) {
  attend_job* j = (attend_job*)arg;
  attend_units(j);
  return NULL;
}

/* Causal (optionally sliding-window, window 0 = full) GQA attention of q
 * [rows][hq d] over the arena; out [rows][hq d]. The (row, head) units are split over
 * `threads` threads as rayon's par_chunks_mut(d) splits them; each unit is serial. */
void orc_attend(const float* q, size_t rows, size_t hq, size_t hkv, size_t d,
                const uint32_t* pos, const uint32_t* pt_off, const uint32_t* pages, size_t page,
                size_t window, const void* kc, const void* vc, int f16, float* out,
                int threads) {
  pthread_once(&g_once, build_table);
  size_t units = rows * hq;
  if (threads < 1) threads = 1;
  if ((size_t)threads > units) threads = (int)(units ? units : 1);
  attend_job* jobs = (attend_job*)calloc((size_t)threads, sizeof(attend_job));
  pthread_t* tids = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
  for (int t = 0; t < threads; ++t) {
    attend_job j = {q, rows, hq, hkv, d, page, window, pos, pt_off, pages, kc, vc, f16, out,
                    units * (size_t)t / (size_t)threads, units * (size_t)(t + 1) / (size_t)threads};
    jobs[t] = j;
  }
  if (threads == 1) {
    attend_units(&jobs[0]);
  } else {
    for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, attend_thread, &jobs[t]);
    for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
  }
  free(jobs);
  free(tids);
}

/* f64 brute force of the same attention (no 16-lane order, f64 exp): the dense
 * reference the f32 restatement is checked against. */
void orc_attend_f64(const float* q, size_t rows, size_t hq, size_t hkv, size_t d,
                    const uint32_t* pos, const uint32_t* pt_off, const uint32_t* pages,
                    size_t page, size_t window, const void* kc, const void* vc, int f16,
                    double* out) {
  pthread_once(&g_once, build_table);
  size_t qd = hq * d, kvd = hkv * d, group = hq / hkv;
  double scale = 1.0 / sqrt((double)d);
  for (size_t i = 0; i < rows; ++i)
    for (size_t h = 0; h < hq; ++h) {
      size_t kh = h / group, p = pos[i], lo = 0;
      if (window) lo = (p + 1 > window) ? p + 1 - window : 0;
      const float* qv = q + i * qd + h * d;
      const uint32_t* pt = pages + pt_off[i];
      double m = -INFINITY;
      double* sc = (double*)malloc(sizeof(double) * (p + 1 - lo));
      for (size_t s = lo; s <= p; ++s) {
        size_t off = ((size_t)pt[s / page] * page + s % page) * kvd + kh * d;
        double acc = 0;
        for (size_t e = 0; e < d; ++e) acc += (double)qv[e] * (double)kv_get(kc, f16, off + e);
        sc[s - lo] = acc * scale;
        if (sc[s - lo] > m) m = sc[s - lo];
      }
      double* o = out + i * qd + h * d;
      for (size_t e = 0; e < d; ++e) o[e] = 0;
      double z = 0;
      for (size_t s = lo; s <= p; ++s) {
        double w = exp(sc[s - lo] - m);
        z += w;
        size_t off = ((size_t)pt[s / page] * page + s % page) * kvd + kh * d;
        for (size_t e = 0; e < d; ++e) o[e] += w * (double)kv_get(vc, f16, off + e);
      }
      for (size_t e = 0; e < d; ++e) o[e] /= z;
      free(sc);
    }
}

/* ---- seeded inputs ------------------------------------------------------------------ */

static uint64_t orc_splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

/* N(0,1) values of stream `seed` from element `offset` (the definition in
 * yaxus_amd/data.py): pair k draws u1, u2 from splitmix64(seed + 2k), (seed + 2k + 1)
 * (top 53 bits), r = sqrt(-2 ln(1 - u1)), th = 2 pi u2; element 2k = r cos th,
 * 2k + 1 = r sin th; f64 math (glibc), rounded to f32. */
void orc_normal(uint64_t seed, uint64_t offset, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) {
    uint64_t e = offset + i, k = e >> 1;
    double u1 = (double)(orc_splitmix64(seed + 2 * k) >> 11) * 0x1.0p-53;
    double u2 = (double)(orc_splitmix64(seed + 2 * k + 1) >> 11) * 0x1.0p-53;
    double r = sqrt(-2.0 * log(1.0 - u1));
    double th = 6.283185307179586 * u2;
    out[i] = (float)((e & 1) ? r * sin(th) : r * cos(th));
  }
}
