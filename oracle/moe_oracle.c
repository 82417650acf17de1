/*
 * CPU restatement of the reference's MoE sparse block: TEST INFRASTRUCTURE ONLY (the parity
 * oracle and the CPU baseline). The header lists what each function follows and how it is pinned.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp), never with -ffast-math: the
 * restatement relies on IEEE f32 semantics with no contraction of a*b+c into fma.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- bf16 ---- */

orc_bf16 orc_bf16_from_f32(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (orc_bf16)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (orc_bf16)(u >> 16);
}

float orc_f32_from_bf16(orc_bf16 h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float R(float f) { return orc_f32_from_bf16(orc_bf16_from_f32(f)); }
static inline float F(orc_bf16 h) { return orc_f32_from_bf16(h); }

void orc_round_bf16_array(const float *in, size_t n, orc_bf16 *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_bf16_from_f32(in[i]);
}

int orc_set_threads(int32_t n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

/* ---- affine dequant (nuvec.rs:602-626, 1173-1204) ---- */

static int qweight_ok(const orc_qweight *w) {
    if (!w || !w->codes) return 0;
    if (w->bits == 16)  /* dense bf16 (SwitchLinear::Dense): no scales */
        return w->experts > 0 && w->out > 0 && w->in > 0 && w->in % 2 == 0;
    if (!w->scales) return 0;
    if (w->bits != 4 && w->bits != 8) return 0;
    if (w->group <= 0 || w->in % w->group != 0) return 0;
    if ((w->in * w->bits) % 32 != 0) return 0;
    return w->experts > 0 && w->out > 0 && w->in > 0;
}

void orc_dequant_row(const orc_qweight *w, int32_t e, int32_t o, float *row) {
    if (w->bits == 16) {  /* dense bf16 experts: the weight itself (gather_mm, nuvec.rs:688-697) */
        const orc_bf16 *d = (const orc_bf16 *)w->codes + ((size_t)e * w->out + o) * (size_t)w->in;
        for (int32_t i = 0; i < w->in; i++) row[i] = F(d[i]);
        return;
    }
    const int per = 32 / w->bits;
    const uint32_t mask = (1u << w->bits) - 1u;
    const size_t words = (size_t)w->in / per;
    const size_t groups = (size_t)w->in / w->group;
    const size_t r = (size_t)e * w->out + o;
    const uint32_t *c = w->codes + r * words;
    const orc_bf16 *s = w->scales + r * groups;
    const orc_bf16 *b = w->biases ? w->biases + r * groups : NULL;
    for (int32_t i = 0; i < w->in; i++) {
        uint32_t q = (c[i / per] >> (w->bits * (i % per))) & mask;
        float scale = F(s[i / w->group]);
        float bias = b ? F(b[i / w->group]) : 0.0f;
        float prod = (float)q * scale;
        row[i] = prod + bias;
    }
}

static float dot_f32(const orc_bf16 *x, const float *w, int32_t n) {
    float acc = 0.0f;
    for (int32_t i = 0; i < n; i++) {
        float p = F(x[i]) * w[i];
        acc = acc + p;
    }
    return acc;
}

/* Pairs grouped by expert (stable): lets each dequantized row serve every pair of its expert. */
typedef struct {
    int32_t n_active;
    int32_t *active;   /* [n_active] expert ids, ascending */
    int32_t *start;    /* [n_active + 1] into list */
    int32_t *list;     /* [n_idx] pair indices */
} groups_t;

static int group_pairs(const uint32_t *idx, int32_t n_idx, int32_t experts, groups_t *g) {
    int32_t *count = calloc((size_t)experts, sizeof(int32_t));
    g->active = malloc(sizeof(int32_t) * (size_t)(experts < n_idx ? experts : n_idx) + 4);
    g->start = malloc(sizeof(int32_t) * ((size_t)(experts < n_idx ? experts : n_idx) + 1) + 4);
    g->list = malloc(sizeof(int32_t) * (size_t)n_idx + 4);
    if (!count || !g->active || !g->start || !g->list) return -1;
    for (int32_t p = 0; p < n_idx; p++) {
        if (idx[p] >= (uint32_t)experts) { free(count); return -1; }
        count[idx[p]]++;
    }
    int32_t n = 0, at = 0;
    int32_t *pos = calloc((size_t)experts, sizeof(int32_t));
    for (int32_t e = 0; e < experts; e++) {
        if (count[e]) {
            g->active[n] = e;
            g->start[n] = at;
            pos[e] = at;
            at += count[e];
            n++;
        }
    }
    g->start[n] = at;
    g->n_active = n;
    for (int32_t p = 0; p < n_idx; p++) g->list[pos[idx[p]]++] = p;
    free(pos);
    free(count);
    return 0;
}

static void free_groups(groups_t *g) {
    free(g->active);
    free(g->start);
    free(g->list);
}

int orc_gather_qmm(const orc_qweight *w, const orc_bf16 *x, int32_t x_rows,
                   const uint32_t *idx, int32_t n_idx, orc_bf16 *y) {
    if (!qweight_ok(w) || !x || !idx || !y || x_rows <= 0 || n_idx <= 0) return -1;
    if (n_idx % x_rows != 0) return -1;
    const int32_t per_x = n_idx / x_rows;
    groups_t g;
    if (group_pairs(idx, n_idx, w->experts, &g) != 0) return -1;
    const int64_t work = (int64_t)g.n_active * w->out;
#pragma omp parallel
    {
        float *row = malloc(sizeof(float) * (size_t)w->in);
#pragma omp for schedule(dynamic, 8)
        for (int64_t it = 0; it < work; it++) {
            int32_t a = (int32_t)(it / w->out), o = (int32_t)(it % w->out);
            orc_dequant_row(w, g.active[a], o, row);
            for (int32_t s = g.start[a]; s < g.start[a + 1]; s++) {
                int32_t p = g.list[s];
                const orc_bf16 *xr = x + (size_t)(p / per_x) * w->in;
                y[(size_t)p * w->out + o] = orc_bf16_from_f32(dot_f32(xr, row, w->in));
            }
        }
        free(row);
    }
    free_groups(&g);
    return 0;
}

int orc_qmatmul(const orc_qweight *w, const orc_bf16 *x, int32_t rows, orc_bf16 *y) {
    if (!w || rows <= 0) return -1;
    uint32_t *idx = calloc((size_t)rows, sizeof(uint32_t));
    if (!idx) return -1;
    int rc = orc_gather_qmm(w, x, rows, idx, rows, y);
    free(idx);
    return rc;
}

int orc_linear_forward(const orc_linear *l, const orc_bf16 *x, int32_t rows, orc_bf16 *y) {
    if (!l || !x || !y || rows <= 0) return -1;
    if (l->dense) {
#pragma omp parallel
        {
            float *row = malloc(sizeof(float) * (size_t)l->in);
#pragma omp for schedule(static)
            for (int32_t o = 0; o < l->out; o++) {
                const orc_bf16 *wr = l->dense + (size_t)o * l->in;
                for (int32_t i = 0; i < l->in; i++) row[i] = F(wr[i]);
                for (int32_t r = 0; r < rows; r++)
                    y[(size_t)r * l->out + o] =
                        orc_bf16_from_f32(dot_f32(x + (size_t)r * l->in, row, l->in));
            }
            free(row);
        }
    } else {
        if (orc_qmatmul(&l->q, x, rows, y) != 0) return -1;
    }
    if (l->bias) {
        for (int64_t i = 0; i < (int64_t)rows * l->out; i++) {
            float s = F(y[i]) + F(l->bias[i % l->out]);
            y[i] = orc_bf16_from_f32(s);
        }
    }
    return 0;
}

/* ---- router ---- */

void orc_softmax(const orc_bf16 *logits, int32_t rows, int32_t n, orc_bf16 *out) {
#pragma omp parallel
    {
        float *e = malloc(sizeof(float) * (size_t)n);
#pragma omp for schedule(static)
        for (int32_t r = 0; r < rows; r++) {
            const orc_bf16 *l = logits + (size_t)r * n;
            float m = -INFINITY;
            for (int32_t i = 0; i < n; i++) m = fmaxf(m, F(l[i]));
            float s = 0.0f;
            for (int32_t i = 0; i < n; i++) {
                e[i] = expf(F(l[i]) - m);
                s = s + e[i];
            }
            for (int32_t i = 0; i < n; i++) out[(size_t)r * n + i] = orc_bf16_from_f32(e[i] / s);
        }
        free(e);
    }
}

/* Rank key: larger gate first, then lower id. Gates are >= 0, so their bf16 bits order them. */
static inline uint32_t rank_key(orc_bf16 g, int32_t id) {
    return ((uint32_t)g << 16) | (uint32_t)(0xffff - id);
}

int orc_topk(const orc_bf16 *gates, int32_t rows, int32_t n, int32_t k, uint32_t *ids) {
    if (k < 1 || k > n || n > 0xffff) return -1;
#pragma omp parallel for schedule(static)
    for (int32_t r = 0; r < rows; r++) {
        const orc_bf16 *g = gates + (size_t)r * n;
        uint32_t prev = 0xffffffffu;
        for (int32_t j = 0; j < k; j++) {
            uint32_t best = 0;
            int32_t best_id = -1;
            for (int32_t i = 0; i < n; i++) {
                uint32_t key = rank_key(g[i], i);
                if (key < prev && (best_id < 0 || key > best)) {
                    best = key;
                    best_id = i;
                }
            }
            ids[(size_t)r * k + j] = (uint32_t)best_id;
            prev = best;
        }
    }
    return 0;
}

void orc_scores(const orc_bf16 *gates, int32_t rows, int32_t n, const uint32_t *ids, int32_t k,
                int32_t norm, orc_bf16 *scores) {
    for (int32_t r = 0; r < rows; r++) {
        for (int32_t j = 0; j < k; j++)
            scores[(size_t)r * k + j] = gates[(size_t)r * n + ids[(size_t)r * k + j]];
        if (norm) {
            float s = 0.0f;
            for (int32_t j = 0; j < k; j++) s = s + F(scores[(size_t)r * k + j]);
            float sum = R(s);
            for (int32_t j = 0; j < k; j++)
                scores[(size_t)r * k + j] = orc_bf16_from_f32(F(scores[(size_t)r * k + j]) / sum);
        }
    }
}

static float bf16_ulp(float v) {
    /* spacing of bf16 values at |v| (the ulp of the binade holding v) */
    float a = fabsf(v);
    if (a == 0.0f) return orc_f32_from_bf16(0x0001);
    int ex;
    frexpf(a, &ex); /* a = m * 2^ex, m in [0.5, 1) */
    float u = ldexpf(1.0f, ex - 8);
    float tiny = orc_f32_from_bf16(0x0001);
    return u > tiny ? u : tiny;
}

int orc_topk_valid(const orc_bf16 *gates, const orc_bf16 *logits, int32_t n, int32_t k,
                   const uint32_t *ids, int32_t ulps) {
    uint32_t own[512];
    if (k > 512 || n > 0xffff) return 0;
    for (int32_t j = 0; j < k; j++) {
        if (ids[j] >= (uint32_t)n) return 0;
        for (int32_t i = 0; i < j; i++)
            if (ids[i] == ids[j]) return 0;
    }
    if (orc_topk(gates, 1, n, k, own) != 0) return 0;
    const uint32_t kth = own[k - 1];
    const float g_b = F(gates[kth]);
    const float l_b = logits ? F(logits[kth]) : 0.0f;
    /* every member of the symmetric difference must tie with the boundary */
    for (int side = 0; side < 2; side++) {
        const uint32_t *a = side ? own : ids, *b = side ? ids : own;
        for (int32_t j = 0; j < k; j++) {
            int found = 0;
            for (int32_t i = 0; i < k; i++) found |= (a[j] == b[i]);
            if (found) continue;
            float g = F(gates[a[j]]);
            if (g == g_b) continue;
            if (logits && ulps > 0) {
                float l = F(logits[a[j]]);
                if (fabsf(l - l_b) <= (float)ulps * bf16_ulp(l_b)) continue;
            }
            return 0;
        }
    }
    return 1;
}

/* ---- dispatch (moe.rs:62-78) ---- */

void orc_floor_divide_u32(const uint32_t *a, size_t n, uint32_t b, uint32_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = a[i] / b;
}

int orc_permute(const uint32_t *ids, int32_t pairs, int32_t k, int32_t experts, uint32_t *order,
                uint32_t *inverse, uint32_t *token, uint32_t *counts) {
    if (!ids || pairs < 0 || k <= 0 || experts <= 0) return -1;
    uint32_t *cnt = calloc((size_t)experts + 1, sizeof(uint32_t));
    if (!cnt) return -1;
    for (int32_t p = 0; p < pairs; p++) {
        if (ids[p] >= (uint32_t)experts) { free(cnt); return -1; }
        cnt[ids[p]]++;
    }
    if (counts) memcpy(counts, cnt, sizeof(uint32_t) * (size_t)experts);
    uint32_t at = 0;
    for (int32_t e = 0; e < experts; e++) {
        uint32_t c = cnt[e];
        cnt[e] = at;
        at += c;
    }
    for (int32_t p = 0; p < pairs; p++) {
        uint32_t pos = cnt[ids[p]]++;
        if (order) order[pos] = (uint32_t)p;
        if (inverse) inverse[p] = pos;
    }
    if (token && order) orc_floor_divide_u32(order, (size_t)pairs, (uint32_t)k, token);
    free(cnt);
    return 0;
}

/* ---- activations and combine ---- */

static inline float sigmoid_f32(float z) { return 1.0f / (1.0f + expf(-z)); }

void orc_swiglu_f32(const float *g, const float *u, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) {
        float s = g[i] * sigmoid_f32(g[i]);
        out[i] = s * u[i];
    }
}

void orc_swiglu(const orc_bf16 *g, const orc_bf16 *u, size_t n, orc_bf16 *out) {
    for (size_t i = 0; i < n; i++) {
        float gv = F(g[i]);
        float s = gv * sigmoid_f32(gv);
        out[i] = orc_bf16_from_f32(s * F(u[i]));
    }
}

void orc_combine(const orc_bf16 *y, const orc_bf16 *scores, int32_t T, int32_t k, int32_t D,
                 orc_bf16 *routed) {
#pragma omp parallel for schedule(static)
    for (int32_t t = 0; t < T; t++) {
        for (int32_t d = 0; d < D; d++) {
            float acc = 0.0f;
            for (int32_t j = 0; j < k; j++) {
                float prod = R(F(y[((size_t)t * k + j) * D + d]) * F(scores[(size_t)t * k + j]));
                acc = acc + prod;
            }
            routed[(size_t)t * D + d] = orc_bf16_from_f32(acc);
        }
    }
}

void orc_shared_add(const orc_bf16 *routed, const orc_bf16 *glogit, const orc_bf16 *shared,
                    int32_t T, int32_t D, orc_bf16 *out, orc_bf16 *gate_out) {
    for (int32_t t = 0; t < T; t++) {
        float sg = R(sigmoid_f32(F(glogit[t])));
        if (gate_out) gate_out[t] = orc_bf16_from_f32(sg);
        for (int32_t d = 0; d < D; d++) {
            size_t i = (size_t)t * D + d;
            float prod = R(sg * F(shared[i]));
            out[i] = orc_bf16_from_f32(F(routed[i]) + prod);
        }
    }
}

void orc_rms_norm(const orc_bf16 *x, const orc_bf16 *w, int32_t rows, int32_t D, float eps,
                  orc_bf16 *y) {
#pragma omp parallel for schedule(static)
    for (int32_t r = 0; r < rows; r++) {
        const orc_bf16 *xr = x + (size_t)r * D;
        float ss = 0.0f;
        for (int32_t d = 0; d < D; d++) {
            float v = F(xr[d]);
            ss = ss + v * v;
        }
        float inv = 1.0f / sqrtf(ss / (float)D + eps);
        for (int32_t d = 0; d < D; d++) {
            float n = R(F(xr[d]) * inv);
            float wv = w ? F(w[d]) : 1.0f;
            y[(size_t)r * D + d] = orc_bf16_from_f32(n * wv);
        }
    }
}

/* ---- the block (moe.rs:149-174) ---- */

static int config_ok(const orc_block *b) {
    const orc_config *c = &b->cfg;
    if (c->hidden <= 0 || c->experts <= 0 || c->intermediate <= 0) return 0;
    if (c->top_k < 1 || c->top_k > c->experts) return 0; /* qwen3_5_moe.rs:508-513 */
    if (!qweight_ok(&b->sw_gate) || !qweight_ok(&b->sw_up) || !qweight_ok(&b->sw_down)) return 0;
    if (b->sw_gate.experts != c->experts || b->sw_gate.out != c->intermediate ||
        b->sw_gate.in != c->hidden)
        return 0;
    if (b->sw_down.out != c->hidden || b->sw_down.in != c->intermediate) return 0;
    if (b->gate.out != c->experts || b->gate.in != c->hidden) return 0;
    return 1;
}

int orc_moe_forward(const orc_block *b, const orc_bf16 *x, int32_t T, orc_bf16 *out,
                    const uint32_t *forced_ids, orc_trace *trace) {
    if (!b || !x || !out || T <= 0 || !config_ok(b)) return -1;
    const orc_config *c = &b->cfg;
    const int32_t D = c->hidden, E = c->experts, k = c->top_k, I = c->intermediate;
    const int32_t P = T * k;
    int rc = -1;

    orc_bf16 *logits = malloc(sizeof(orc_bf16) * (size_t)T * E);
    orc_bf16 *gates = malloc(sizeof(orc_bf16) * (size_t)T * E);
    uint32_t *ids = malloc(sizeof(uint32_t) * (size_t)P);
    orc_bf16 *scores = malloc(sizeof(orc_bf16) * (size_t)P);
    uint32_t *order = malloc(sizeof(uint32_t) * (size_t)P);
    uint32_t *inverse = malloc(sizeof(uint32_t) * (size_t)P);
    uint32_t *token = malloc(sizeof(uint32_t) * (size_t)P);
    uint32_t *idx = malloc(sizeof(uint32_t) * (size_t)P);
    orc_bf16 *rows = malloc(sizeof(orc_bf16) * (size_t)P * D);
    orc_bf16 *up = malloc(sizeof(orc_bf16) * (size_t)P * I);
    orc_bf16 *gt = malloc(sizeof(orc_bf16) * (size_t)P * I);
    orc_bf16 *act = malloc(sizeof(orc_bf16) * (size_t)P * I);
    orc_bf16 *ys = malloc(sizeof(orc_bf16) * (size_t)P * D);
    orc_bf16 *y = malloc(sizeof(orc_bf16) * (size_t)P * D);
    orc_bf16 *routed = malloc(sizeof(orc_bf16) * (size_t)T * D);
    if (!logits || !gates || !ids || !scores || !order || !inverse || !token || !idx || !rows ||
        !up || !gt || !act || !ys || !y || !routed)
        goto done;

    /* router: gates = softmax(gate(x)); top-k; scores (moe.rs:151-159) */
    if (orc_linear_forward(&b->gate, x, T, logits) != 0) goto done;
    orc_softmax(logits, T, E, gates);
    if (forced_ids) {
        for (int32_t t = 0; t < T; t++) {
            if (!orc_topk_valid(gates + (size_t)t * E, logits + (size_t)t * E, E, k,
                                forced_ids + (size_t)t * k, 1)) {
                rc = -2;
                goto done;
            }
        }
        memcpy(ids, forced_ids, sizeof(uint32_t) * (size_t)P);
    } else if (orc_topk(gates, T, E, k, ids) != 0) {
        goto done;
    }
    orc_scores(gates, T, E, ids, k, c->norm_topk_prob, scores);

    /* SwitchGlu (moe.rs:61-94) */
    const int sorted = P >= 64; /* SORT_AT */
    if (sorted) {
        if (orc_permute(ids, P, k, E, order, inverse, token, NULL) != 0) goto done;
        for (int32_t i = 0; i < P; i++) {
            memcpy(rows + (size_t)i * D, x + (size_t)token[i] * D, sizeof(orc_bf16) * (size_t)D);
            idx[i] = ids[order[i]];
        }
        if (orc_gather_qmm(&b->sw_up, rows, P, idx, P, up) != 0) goto done;
        if (orc_gather_qmm(&b->sw_gate, rows, P, idx, P, gt) != 0) goto done;
        orc_swiglu(gt, up, (size_t)P * I, act);
        if (orc_gather_qmm(&b->sw_down, act, P, idx, P, ys) != 0) goto done;
        /* y = take(y, inverse): pair p's output sits at sorted position inverse[p] */
        for (int32_t p = 0; p < P; p++)
            memcpy(y + (size_t)p * D, ys + (size_t)inverse[p] * D, sizeof(orc_bf16) * (size_t)D);
        if (trace && trace->act)
            for (int32_t p = 0; p < P; p++)
                memcpy(trace->act + (size_t)p * I, act + (size_t)inverse[p] * I,
                       sizeof(orc_bf16) * (size_t)I);
    } else {
        if (orc_gather_qmm(&b->sw_up, x, T, ids, P, up) != 0) goto done;
        if (orc_gather_qmm(&b->sw_gate, x, T, ids, P, gt) != 0) goto done;
        orc_swiglu(gt, up, (size_t)P * I, act);
        if (orc_gather_qmm(&b->sw_down, act, P, ids, P, y) != 0) goto done;
        if (trace && trace->act) memcpy(trace->act, act, sizeof(orc_bf16) * (size_t)P * I);
    }
    orc_combine(y, scores, T, k, D, routed);

    /* shared expert under a sigmoid gate (moe.rs:166-171) */
    if (c->shared_intermediate > 0) {
        const int32_t S = c->shared_intermediate;
        orc_bf16 *gl = malloc(sizeof(orc_bf16) * (size_t)T);
        orc_bf16 *sg = malloc(sizeof(orc_bf16) * (size_t)T * S);
        orc_bf16 *su = malloc(sizeof(orc_bf16) * (size_t)T * S);
        orc_bf16 *sa = malloc(sizeof(orc_bf16) * (size_t)T * S);
        orc_bf16 *sy = malloc(sizeof(orc_bf16) * (size_t)T * D);
        int ok = gl && sg && su && sa && sy &&
                 orc_linear_forward(&b->sh_expert_gate, x, T, gl) == 0 &&
                 orc_linear_forward(&b->sh_gate, x, T, sg) == 0 &&
                 orc_linear_forward(&b->sh_up, x, T, su) == 0;
        if (ok) {
            orc_swiglu(sg, su, (size_t)T * S, sa);
            ok = orc_linear_forward(&b->sh_down, sa, T, sy) == 0;
        }
        if (ok) {
            orc_shared_add(routed, gl, sy, T, D, out, trace ? trace->shared_gate : NULL);
            if (trace && trace->shared_y) memcpy(trace->shared_y, sy, sizeof(orc_bf16) * (size_t)T * D);
        }
        free(gl);
        free(sg);
        free(su);
        free(sa);
        free(sy);
        if (!ok) goto done;
    } else {
        memcpy(out, routed, sizeof(orc_bf16) * (size_t)T * D);
    }

    if (trace) {
        if (trace->logits) memcpy(trace->logits, logits, sizeof(orc_bf16) * (size_t)T * E);
        if (trace->gates) memcpy(trace->gates, gates, sizeof(orc_bf16) * (size_t)T * E);
        if (trace->ids) memcpy(trace->ids, ids, sizeof(uint32_t) * (size_t)P);
        if (trace->scores) memcpy(trace->scores, scores, sizeof(orc_bf16) * (size_t)P);
        if (trace->order && sorted) memcpy(trace->order, order, sizeof(uint32_t) * (size_t)P);
        if (trace->inverse && sorted) memcpy(trace->inverse, inverse, sizeof(uint32_t) * (size_t)P);
        if (trace->y) memcpy(trace->y, y, sizeof(orc_bf16) * (size_t)P * D);
        if (trace->routed) memcpy(trace->routed, routed, sizeof(orc_bf16) * (size_t)T * D);
    }
    rc = 0;
done:
    free(logits);
    free(gates);
    free(ids);
    free(scores);
    free(order);
    free(inverse);
    free(token);
    free(idx);
    free(rows);
    free(up);
    free(gt);
    free(act);
    free(ys);
    free(y);
    free(routed);
    return rc;
}

/* ---- the block in f32 (an f32 checkpoint: moe.rs:149-174 with no bf16 rounding) ---- */

static float dot32(const float *a, const float *w, int32_t n) {
    float acc = 0.0f;
    for (int32_t i = 0; i < n; i++) acc = acc + a[i] * w[i];
    return acc;
}

int orc_moe_forward_f32(const orc_block_f32 *b, const float *x, int32_t T, float *out,
                        uint32_t *ids_out) {
    if (!b || !x || !out || T <= 0) return -1;
    const orc_config *c = &b->cfg;
    const int32_t D = c->hidden, E = c->experts, k = c->top_k, I = c->intermediate;
    const int32_t S = c->shared_intermediate;
    if (D <= 0 || E <= 0 || I <= 0 || k < 1 || k > E || S < 0) return -1;
    if (!b->router || !b->sw_gate || !b->sw_up || !b->sw_down) return -1;
    if (S > 0 && (!b->sh_gate || !b->sh_up || !b->sh_down || !b->sh_expert_gate)) return -1;
    int rc = 0;
#pragma omp parallel for schedule(dynamic)
    for (int32_t t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * D;
        float *gates = malloc(sizeof(float) * (size_t)E);
        int *taken = calloc((size_t)E, sizeof(int));
        float *act = malloc(sizeof(float) * (size_t)(I > S ? I : S));
        float *acc = malloc(sizeof(float) * (size_t)D);
        uint32_t ids[64];
        float sc[64];
        if (!gates || !taken || !act || !acc || k > 64) {
#pragma omp atomic write
            rc = -1;
            free(gates), free(taken), free(act), free(acc);
            continue;
        }
        /* router: softmax(x W^T) over the experts (moe.rs:151-155) */
        float m = -INFINITY, sum = 0.0f;
        for (int32_t e = 0; e < E; e++) {
            gates[e] = dot32(xt, b->router + (size_t)e * D, D);
            m = gates[e] > m ? gates[e] : m;
        }
        for (int32_t e = 0; e < E; e++) {
            gates[e] = expf(gates[e] - m);
            sum = sum + gates[e];
        }
        for (int32_t e = 0; e < E; e++) gates[e] = gates[e] / sum;
        /* top-k in rank order, equal gates by lower id; scores (moe.rs:156-159) */
        float tot = 0.0f;
        for (int32_t j = 0; j < k; j++) {
            int32_t best = -1;
            for (int32_t e = 0; e < E; e++)
                if (!taken[e] && (best < 0 || gates[e] > gates[best])) best = e;
            taken[best] = 1;
            ids[j] = (uint32_t)best;
            sc[j] = gates[best];
            tot = tot + sc[j];
        }
        if (c->norm_topk_prob)
            for (int32_t j = 0; j < k; j++) sc[j] = sc[j] / tot;
        /* experts: y = down(silu(gate x) * up x); routed = sum_j y_j * score_j (moe.rs:79-94,
           160-165) */
        for (int32_t d = 0; d < D; d++) acc[d] = 0.0f;
        for (int32_t j = 0; j < k; j++) {
            const size_t e = ids[j];
            for (int32_t i = 0; i < I; i++) {
                float g = dot32(xt, b->sw_gate + (e * I + i) * D, D);
                float u = dot32(xt, b->sw_up + (e * I + i) * D, D);
                act[i] = (g * sigmoid_f32(g)) * u;
            }
            for (int32_t d = 0; d < D; d++)
                acc[d] = acc[d] + dot32(act, b->sw_down + (e * D + d) * I, I) * sc[j];
        }
        /* the shared expert under its sigmoid gate (moe.rs:166-171) */
        if (S > 0) {
            float sg = sigmoid_f32(dot32(xt, b->sh_expert_gate, D));
            for (int32_t i = 0; i < S; i++) {
                float g = dot32(xt, b->sh_gate + (size_t)i * D, D);
                float u = dot32(xt, b->sh_up + (size_t)i * D, D);
                act[i] = (g * sigmoid_f32(g)) * u;
            }
            for (int32_t d = 0; d < D; d++)
                acc[d] = acc[d] + sg * dot32(act, b->sh_down + (size_t)d * S, S);
        }
        memcpy(out + (size_t)t * D, acc, sizeof(float) * (size_t)D);
        if (ids_out) memcpy(ids_out + (size_t)t * k, ids, sizeof(uint32_t) * (size_t)k);
        free(gates), free(taken), free(act), free(acc);
    }
    return rc;
}

int orc_moe_stack(const orc_block *blocks, int32_t n_layers, const orc_bf16 *norm_w, float eps,
                  orc_bf16 *x, int32_t T) {
    if (!blocks || n_layers <= 0 || !x || T <= 0) return -1;
    const int32_t D = blocks[0].cfg.hidden;
    orc_bf16 *h = malloc(sizeof(orc_bf16) * (size_t)T * D);
    orc_bf16 *o = malloc(sizeof(orc_bf16) * (size_t)T * D);
    int rc = (h && o) ? 0 : -1;
    for (int32_t l = 0; rc == 0 && l < n_layers; l++) {
        orc_rms_norm(x, norm_w ? norm_w + (size_t)l * D : NULL, T, D, eps, h);
        rc = orc_moe_forward(&blocks[l], h, T, o, NULL, NULL);
        if (rc == 0)
            for (size_t i = 0; i < (size_t)T * D; i++) x[i] = orc_bf16_from_f32(F(x[i]) + F(o[i]));
    }
    free(h);
    free(o);
    return rc;
}
