/*
 * kvref — CPU restatement of the reference INT8 KV-cache semantics.
 * TEST INFRASTRUCTURE ONLY (the checker, never the product). See kvref.h for the
 * per-function reference citations and what pins each function.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off; no fast-math, so every
 * float expression below is a single IEEE round-to-nearest operation).
 */
#include "kvref.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

uint64_t kvref_value_index(uint32_t vector, uint32_t dimension) {
    /* kernels.metal:126-128: token=vector/2, head=vector%2;
     * ((token/256)*2+head)*65536 + dimension*256 + token%256 */
    uint64_t token = vector / 2u, head = vector % 2u;
    return ((token / 256u) * 2u + head) * 65536u + (uint64_t)dimension * 256u + token % 256u;
}

uint64_t kvref_value_bytes(uint32_t length) {
    /* Int8KvTests.cs:11: ((length+255)/256*256)*512 */
    return ((uint64_t)length + 255u) / 256u * 256u * 512u;
}

void kvref_quantize(const float *x, int8_t *codes, float *scale) {
    /* kernels.metal:135-140 / Int8KvTests.cs:116-118 */
    float amax = 0.0f;
    for (int d = 0; d < 256; d++) {
        float a = fabsf(x[d]);
        if (a > amax) amax = a;
    }
    volatile float s = amax / 127.0f;          /* fp32 RN division */
    *scale = s;
    if (!(amax > 0.0f)) {
        for (int d = 0; d < 256; d++) codes[d] = 0;
        return;
    }
    volatile float r = 127.0f / amax;          /* fp32 RN division */
    for (int d = 0; d < 256; d++) {
        volatile float p = x[d] * r;           /* one fp32 RN multiply */
        float c = rintf(p);                    /* default mode: round half to even */
        if (c > 127.0f) c = 127.0f;
        if (c < -127.0f) c = -127.0f;
        codes[d] = (int8_t)c;
    }
}

void kvref_store(const float *k, const float *v, int rows, int pos,
                 int8_t *kc, int8_t *vc, float *ks, float *vs) {
    int8_t codes[256];
    float scale;
    for (int row = 0; row < rows; row++) {
        for (int h = 0; h < 2; h++) {
            uint32_t vector = (uint32_t)(pos + row) * 2u + (uint32_t)h;
            kvref_quantize(k + ((size_t)row * 2 + h) * 256, codes, &scale);
            ks[vector] = scale;
            memcpy(kc + (size_t)vector * 256, codes, 256);
            kvref_quantize(v + ((size_t)row * 2 + h) * 256, codes, &scale);
            vs[vector] = scale;
            for (int d = 0; d < 256; d++) vc[kvref_value_index(vector, (uint32_t)d)] = codes[d];
        }
    }
}

typedef struct {
    const float *k, *v;
    int rows, pos, first, count;
    int8_t *kc, *vc;
    float *ks, *vs;
} store_job;

static void *store_worker(void *arg) {
    store_job *j = (store_job *)arg;
    kvref_store(j->k + (size_t)j->first * 512, j->v + (size_t)j->first * 512, j->count, j->pos + j->first,
                j->kc, j->vc, j->ks, j->vs);
    return NULL;
}

void kvref_store_mt(const float *k, const float *v, int rows, int pos,
                    int8_t *kc, int8_t *vc, float *ks, float *vs, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if (threads > rows) threads = rows > 0 ? rows : 1;
    store_job jobs[256];
    pthread_t tid[256];
    int started[256];
    int per = (rows + threads - 1) / threads;
    for (int i = 0; i < threads; i++) {
        int first = i * per, count = rows - first < per ? rows - first : per;
        if (count < 0) count = 0;
        jobs[i] = (store_job){k, v, rows, pos, first, count, kc, vc, ks, vs};
        started[i] = i > 0 && count > 0 && pthread_create(&tid[i], NULL, store_worker, &jobs[i]) == 0;
        if (i > 0 && count > 0 && !started[i]) store_worker(&jobs[i]);
    }
    if (jobs[0].count > 0) store_worker(&jobs[0]);
    for (int i = 1; i < threads; i++)
        if (started[i]) pthread_join(tid[i], NULL);
}

double kvref_rotate_f64(const float *x, int d, int position) {
    /* Int8KvTests.cs:13-18 */
    if (d >= 64) return x[d];
    int j = d % 32;
    double angle = position * pow(10000000.0, -2.0 * j / 64);
    return d < 32 ? x[j] * cos(angle) - x[j + 32] * sin(angle)
                  : x[j + 32] * cos(angle) + x[j] * sin(angle);
}

uint16_t kvref_half_bits(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);      /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                        /* below 2^-14: subnormal */
        float a;
        memcpy(&a, &ax, 4);
        return (uint16_t)(sign | (uint32_t)rintf(a * 16777216.0f)); /* exact scale, RNE */
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float kvref_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u, x;
    if (e == 0) {
        float r = (float)m * (1.0f / 16777216.0f);
        return (h & 0x8000u) ? -r : r;
    }
    if (e == 31) x = sign | 0x7f800000u | (m << 13);
    else x = sign | ((e + 112u) << 23) | (m << 13);
    float r;
    memcpy(&r, &x, 4);
    return r;
}

float kvref_bf16_round(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) x |= 0x00400000u;   /* quiet NaN */
    else x += 0x7fffu + ((x >> 16) & 1u);
    x &= 0xffff0000u;
    float r;
    memcpy(&r, &x, 4);
    return r;
}

void kvref_query_grouped_half(const float *x, int rows, int group, uint16_t *y) {
    /* kernels.metal:1276-1281: logical=at/256, block=logical/(M*A), local=logical%(M*A),
     * row=local/A, head=block*A+local%A; y[at]=half(x[(row*16+head)*256+d]) */
    for (int64_t logical = 0; logical < (int64_t)rows * 16; logical++) {
        int64_t block = logical / ((int64_t)rows * group), local = logical % ((int64_t)rows * group);
        int64_t row = local / group, head = block * group + local % group;
        for (int d = 0; d < 256; d++) y[logical * 256 + d] = kvref_half_bits(x[(row * 16 + head) * 256 + d]);
    }
}

/* ---------------------------------------------------------------- attention */

typedef struct {
    const float *q;
    int round_q_half;
    const int8_t *kc, *vc;
    const float *ks, *vs, *gate;
    const uint16_t *kh, *vh;   /* FP16 control cache when non-NULL */
    int rows, pos;
    double *out, *bound;
    int64_t next, total;       /* work items = rows*16 */
    pthread_mutex_t lock;
} attn_job;

static void attend_one(attn_job *j, int row, int head, double *logits) {
    int length = j->pos + row + 1, g = head / 8;
    double q[256];
    for (int d = 0; d < 256; d++) {
        float value = j->q[((size_t)row * 16 + head) * 256 + d];
        q[d] = j->round_q_half ? (double)kvref_half_to_float(kvref_half_bits(value)) : (double)value;
    }
    double maxv = -INFINITY;
    for (int t = 0; t < length; t++) {
        double acc = 0;
        size_t at = ((size_t)t * 2 + g) * 256;
        if (j->kh) {
            for (int d = 0; d < 256; d++) acc += q[d] * (double)kvref_half_to_float(j->kh[at + d]) / 16;
        } else {
            /* Int8KvTests.cs:137: query * code * ks / 16, accumulated in FP64 */
            double ks = j->ks[(size_t)t * 2 + g];
            for (int d = 0; d < 256; d++) acc += q[d] * j->kc[at + d] * ks / 16;
        }
        logits[t] = acc;
        if (acc > maxv) maxv = acc;
    }
    double sum = 0;
    for (int t = 0; t < length; t++) {
        logits[t] = exp(logits[t] - maxv);
        sum += logits[t];
    }
    double *o = j->out + ((size_t)row * 16 + head) * 256;
    double *b = j->bound ? j->bound + ((size_t)row * 16 + head) * 256 : NULL;
    double acc[256], mag[256];
    for (int d = 0; d < 256; d++) acc[d] = mag[d] = 0;
    for (int t = 0; t < length; t++) {
        double p = logits[t] / sum;
        uint32_t vector = (uint32_t)t * 2u + (uint32_t)g;
        if (j->vh) {
            for (int d = 0; d < 256; d++) acc[d] += p * (double)kvref_half_to_float(j->vh[(size_t)vector * 256 + d]);
        } else {
            /* Int8KvTests.cs:147: exp/sum * vcode * vs */
            double vs = j->vs[vector];
            uint64_t page = kvref_value_index(vector, 0);
            for (int d = 0; d < 256; d++) {
                double c = p * j->vc[page + (uint64_t)d * 256u] * vs;
                acc[d] += c;
                mag[d] += fabs(c);
            }
        }
    }
    for (int d = 0; d < 256; d++) {
        /* Int8KvTests.cs:151-152: expected / (1 + exp(-gate)) */
        double gv = 1.0 + exp(-(double)j->gate[((size_t)row * 16 + head) * 256 + d]);
        o[d] = acc[d] / gv;
        if (b) b[d] = mag[d] / gv;
    }
}

static void *attn_worker(void *arg) {
    attn_job *j = (attn_job *)arg;
    double *logits = (double *)malloc(sizeof(double) * ((size_t)j->pos + j->rows + 1));
    for (;;) {
        pthread_mutex_lock(&j->lock);
        int64_t item = j->next++;
        pthread_mutex_unlock(&j->lock);
        if (item >= j->total) break;
        attend_one(j, (int)(item / 16), (int)(item % 16), logits);
    }
    free(logits);
    return NULL;
}

static void run_attention(attn_job *j, int threads) {
    j->next = 0;
    j->total = (int64_t)j->rows * 16;
    pthread_mutex_init(&j->lock, NULL);
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    int started = 0;
    for (int i = 1; i < threads; i++)
        if (pthread_create(&tid[started], NULL, attn_worker, j) == 0) started++;
    attn_worker(j);
    for (int i = 0; i < started; i++) pthread_join(tid[i], NULL);
    pthread_mutex_destroy(&j->lock);
}

void kvref_attention_f64(const float *q, int round_q_half,
                         const int8_t *kc, const int8_t *vc,
                         const float *ks, const float *vs, const float *gate,
                         int rows, int pos, double *out, double *bound, int threads) {
    attn_job j;
    memset(&j, 0, sizeof j);
    j.q = q; j.round_q_half = round_q_half; j.kc = kc; j.vc = vc; j.ks = ks; j.vs = vs;
    j.gate = gate; j.rows = rows; j.pos = pos; j.out = out; j.bound = bound;
    run_attention(&j, threads);
}

void kvref_attention_fp16kv_f64(const float *q, int round_q_half,
                                const uint16_t *kh, const uint16_t *vh, const float *gate,
                                int rows, int pos, double *out, int threads) {
    attn_job j;
    memset(&j, 0, sizeof j);
    j.q = q; j.round_q_half = round_q_half; j.kh = kh; j.vh = vh;
    j.gate = gate; j.rows = rows; j.pos = pos; j.out = out;
    run_attention(&j, threads);
}

/* ---------------------------------------------------------------- online emulator */

typedef struct {
    const float *q;
    const int8_t *kc, *vc;
    const float *ks, *vs, *gate;
    int rows, pos, tile_keys, p_mode;
    float *out;
    int64_t next, total;
    pthread_mutex_t lock;
} online_job;

static float sigmoid_f32(float g) {
    volatile float e = expf(-g);
    volatile float d = 1.0f + e;
    return 1.0f / d;
}

/* One (row, head) of the reference's tuned online INT8 prefill, kernels.metal:1378-1457,
 * with its roundings: FP16 query (:1276-1281); per 256-key tile the FP32 score
 * (q16 . code) scaled as (s * (1/16)) * ks (:1419-1421), masked beyond pos + row; the tile
 * maximum joins the running one (:1424), decay = exp(old - new) and the unscaled exponentials
 * exp(a - new) in FP32 (:1425-1426); the probability operand P = bfloat(e * vs) (:1427);
 * the denominator sums the unrounded e (:1428-1429); the accumulator is scaled by the decay
 * (:1436-1437) and gains sum_t P_t * vcode_t (BF16 x INT8 products are exact; the tile's sum
 * is rounded to FP32 once, :1438-1447); y = out / denominator * sigmoid(gate) (:1452-1453).
 * The FP32 dot products and tile sums are formed in FP64 and rounded once (the matrix units'
 * summation order is not observable here); exp is the C library's expf.
 * p_mode 1 replaces (:1427) by this build's rounding, FP16(e * (vs / vs_ref)) with vs_ref the
 * largest V scale over the attended keys, and multiplies vs_ref back at the end;
 * p_mode 2 keeps P = e * vs in FP32 (no operand rounding);
 * p_mode 3 is this build's current form: P = FP16(e * r) with r = 2^7 vs / vs_ref (2^7 for a
 * zero V vector), the denominator sums P * (1 / r) (the rounded operand divided back by its
 * factor) instead of e, and vs_ref / 2^7 multiplies the result at the end. */
static void online_one(online_job *j, int row, int head, float *vals) {
    const int g = head / 8, length = j->pos + row + 1, T = j->tile_keys;
    float q[256];
    for (int d = 0; d < 256; d++)
        q[d] = kvref_half_to_float(kvref_half_bits(j->q[((size_t)row * 16 + head) * 256 + d]));
    float vs_ref = 0.0f;
    for (int t = 0; t < length; t++) {
        float v = j->vs[(size_t)t * 2 + g];
        if (v > vs_ref) vs_ref = v;
    }
    volatile float vs_inv = vs_ref > 0.0f ? 1.0f / vs_ref : 0.0f;
    float out[256];
    for (int d = 0; d < 256; d++) out[d] = 0.0f;
    float maximum = -INFINITY, denominator = 0.0f;
    for (int key = 0; key < length; key += T) {
        int n = length - key < T ? length - key : T;
        float top = -INFINITY;
        for (int i = 0; i < n; i++) {
            int t = key + i;
            const int8_t *k = j->kc + ((size_t)t * 2 + g) * 256;
            double dot = 0;
            for (int d = 0; d < 256; d++) dot += (double)q[d] * (double)k[d];
            volatile float s = (float)dot;
            volatile float a = s * (1.0f / 16.0f);
            volatile float b = a * j->ks[(size_t)t * 2 + g];
            vals[i] = b;
            if (b > top) top = b;
        }
        float next = maximum > top ? maximum : top;
        volatile float decay = expf(maximum - next);
        float total = 0.0f;
        double tile[256];
        for (int d = 0; d < 256; d++) tile[d] = 0;
        for (int i = 0; i < n; i++) {
            int t = key + i;
            volatile float value = expf(vals[i] - next);
            float vsc = j->vs[(size_t)t * 2 + g];
            float p;
            if (j->p_mode == 0) {
                volatile float scaled = value * vsc;
                p = kvref_bf16_round(scaled);
            } else if (j->p_mode == 1) {
                volatile float ratio = vsc * vs_inv;
                volatile float scaled = value * ratio;
                p = kvref_half_to_float(kvref_half_bits(scaled));
            } else if (j->p_mode == 3) {
                volatile float ratio = vsc * vs_inv;
                volatile float r = vsc > 0.0f ? ratio * 128.0f : 128.0f;
                volatile float scaled = value * r;
                volatile float inverse = 1.0f / r;
                p = kvref_half_to_float(kvref_half_bits(scaled));
                volatile float weight = p * inverse;
                value = weight;   /* the denominator takes the rounded operand, divided back */
            } else {
                volatile float scaled = value * vsc;
                p = scaled;
            }
            total += value;
            uint64_t page = kvref_value_index((uint32_t)t * 2u + (uint32_t)g, 0);
            for (int d = 0; d < 256; d++) tile[d] += (double)p * (double)j->vc[page + (uint64_t)d * 256u];
        }
        volatile float scaled_denominator = denominator * decay;
        denominator = scaled_denominator + total;
        maximum = next;
        for (int d = 0; d < 256; d++) {
            volatile float kept = out[d] * decay;
            volatile float gained = (float)tile[d];
            out[d] = kept + gained;
        }
    }
    float *y = j->out + ((size_t)row * 16 + head) * 256;
    for (int d = 0; d < 256; d++) {
        volatile float o = j->p_mode == 1 ? out[d] * vs_ref : j->p_mode == 3 ? out[d] * (vs_ref / 128.0f) : out[d];
        volatile float r = o / denominator;
        y[d] = r * sigmoid_f32(j->gate[((size_t)row * 16 + head) * 256 + d]);
    }
}

static void *online_worker(void *arg) {
    online_job *j = (online_job *)arg;
    float *vals = (float *)malloc(sizeof(float) * (size_t)j->tile_keys);
    for (;;) {
        pthread_mutex_lock(&j->lock);
        int64_t item = j->next++;
        pthread_mutex_unlock(&j->lock);
        if (item >= j->total) break;
        online_one(j, (int)(item / 16), (int)(item % 16), vals);
    }
    free(vals);
    return NULL;
}

void kvref_attention_online_emulate(const float *q, const int8_t *kc, const int8_t *vc,
                                    const float *ks, const float *vs, const float *gate,
                                    int rows, int pos, int tile_keys, int p_mode,
                                    float *out, int threads) {
    online_job j;
    memset(&j, 0, sizeof j);
    j.q = q; j.kc = kc; j.vc = vc; j.ks = ks; j.vs = vs; j.gate = gate;
    j.rows = rows; j.pos = pos; j.tile_keys = tile_keys > 0 ? tile_keys : 256; j.p_mode = p_mode;
    j.out = out; j.next = 0; j.total = (int64_t)rows * 16;
    pthread_mutex_init(&j.lock, NULL);
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    int started = 0;
    for (int i = 1; i < threads; i++)
        if (pthread_create(&tid[started], NULL, online_worker, &j) == 0) started++;
    online_worker(&j);
    for (int i = 0; i < started; i++) pthread_join(tid[i], NULL);
    pthread_mutex_destroy(&j.lock);
}

/* ---------------------------------------------------------------- generators */

void kvref_fill_hash(float *out, int64_t count, uint32_t seed, float scale) {
    /* FastAttentionTests.cs:111-119 */
    for (int64_t i = 0; i < count; i++) {
        uint32_t h = (uint32_t)i + seed * 0x9e3779b9u;
        h ^= h >> 16;
        h *= 0x7feb352du;
        h ^= h >> 15;
        volatile float centered = (float)(h & 65535u) - 32768.0f;
        volatile float unit = centered / 49157.0f;
        out[i] = unit * scale;
    }
}

static uint64_t splitmix64(uint64_t *state) {
    uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

void kvref_splitmix64(uint64_t seed, uint64_t *out, int64_t count) {
    uint64_t state = seed;
    for (int64_t i = 0; i < count; i++) out[i] = splitmix64(&state);
}

static double uniform01(uint64_t *state) {
    return ((double)(splitmix64(state) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

static void normal_pair(uint64_t *state, double *a, double *b) {
    double u1 = uniform01(state), u2 = uniform01(state);
    double r = sqrt(-2.0 * log(u1)), th = 6.283185307179586476925286766559 * u2;
    *a = r * cos(th);
    *b = r * sin(th);
}

void kvref_normal(float *out, int64_t count, uint64_t seed) {
    uint64_t state = seed;
    for (int64_t i = 0; i < count; i += 2) {
        double a, b;
        normal_pair(&state, &a, &b);
        out[i] = (float)a;
        if (i + 1 < count) out[i + 1] = (float)b;
    }
}

void kvref_student_t4(float *out, int64_t count, uint64_t seed) {
    uint64_t state = seed;
    for (int64_t i = 0; i < count; i++) {
        double n[6];
        normal_pair(&state, &n[0], &n[1]);
        normal_pair(&state, &n[2], &n[3]);
        normal_pair(&state, &n[4], &n[5]);
        double chi2 = n[1] * n[1] + n[2] * n[2] + n[3] * n[3] + n[4] * n[4];
        out[i] = (float)(n[0] / sqrt(chi2 / 4.0));
    }
}
