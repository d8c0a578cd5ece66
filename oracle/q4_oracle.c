/*
 * q4_oracle.c -- CPU restatement of qw's int4 ("q4") matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker that the HIP kernels are
 * compared against; it is loaded by tests/, by __graft_entry__.smoke() and by
 * bench.py's cpu_baseline leg, and never by the product library.
 *
 * What it restates (reference paths relative to the reference repository):
 *   - number conversions           src/core/common.hpp:34-99
 *   - int4 g128 unpack / dequant   src/ref/ref_model.cpp:100-119, docs/MODEL.md:34-37
 *       generalised with a per-group 4-bit zero point z: w = (q - z) * s.
 *       With no zero array z == 8, which is the reference's symmetric format.
 *   - expert_linear (fp32 dot)      src/ref/ref_model.cpp:25-30, 100-119
 *   - engine nibble order          src/engine/weight_convert.cpp:61-71
 *   - int4 g128 quantiser          src/engine/weight_convert.cpp:73-90
 *   - MoE routing and combine      src/ref/ref_model.cpp:406-463
 *   - 16-bit dense linear          src/ref/ref_model.cpp:86-97
 *   - shared expert (SwiGLU, gate) src/ref/ref_model.cpp:465-478
 *   - slot order                   src/kernels/moe_route.hip:149-160
 *   - W4A8 expert GEMMs (opt-in)   src/kernels/moe_w4a8.hip:13-215
 *   - int8 dense rows (i8 GEMV)    src/engine/weight_convert.cpp:92-108,
 *                                  src/kernels/gemv.hip:75-136
 *   - parallel_for chunking        src/core/threadpool.hpp:38-58
 *
 * Formats used throughout (the device formats of this build):
 *   W  uint32 [N][K/8]        element 8c+i of a row at bits 4i of word c
 *   S  fp16   [N][K/128]      one scale per 128-weight group along K
 *   Z  uint32 [N][ceil(G/8)]  4-bit zero of group g at bits 4(g%8) of word g/8;
 *                             NULL means z = 8 for every group
 *
 * Parity pinning (what each function is checked against) is listed in the
 * test files tests/test_oracle*.py; every function here has at least one
 * check that does not retype its formula.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QGROUP 128

/* ---------------------------------------------------------------- numbers */

/* src/core/common.hpp:34-39: bf16 is the top half of an fp32. */
float o_bf16_to_f32(uint16_t v) {
    uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* src/core/common.hpp:41-65: exact fp16 -> fp32, subnormals renormalised. */
float o_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, u;
    if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else {
            exp = 127 - 15 + 1;
            while (!(man & 0x400u)) {
                man <<= 1;
                --exp;
            }
            man &= 0x3ffu;
            u = sign | (exp << 23) | (man << 13);
        }
    } else if (exp == 31) {
        u = sign | 0x7f800000u | (man << 13);
    } else {
        u = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* src/core/common.hpp:76-97: round-to-nearest-even fp32 -> fp16. */
uint16_t o_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    int32_t exp = (int32_t)((u >> 23) & 0xffu) - 127 + 15;
    uint32_t man = u & 0x7fffffu;
    if (((u >> 23) & 0xffu) == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    if (exp >= 31) return (uint16_t)(sign | 0x7c00u);
    if (exp <= 0) {
        if (exp < -10) return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - exp);
        uint32_t half = man >> shift, rem = man & ((1u << shift) - 1u), mid = 1u << (shift - 1);
        if (rem > mid || (rem == mid && (half & 1u))) ++half;
        return (uint16_t)(sign | half);
    }
    uint32_t half = sign | ((uint32_t)exp << 10) | (man >> 13), rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) ++half;
    return (uint16_t)half;
}

/* src/engine/weight_convert.cpp:19-26: bf16 -> fp16 at load, magnitudes above
 * the fp16 maximum saturated to +-65504 (infinities too; NaN stays NaN). */
uint16_t o_bf16_to_f16(uint16_t b) {
    float f = o_bf16_to_f32(b);
    if (fabsf(f) > 65504.f) f = f > 0 ? 65504.f : -65504.f;
    return o_f32_to_f16(f);
}

/* Round-to-nearest-even fp32 -> bf16 (NaN kept quiet). The reference has no
 * bf16 writer (gfx1030 has no bf16); this is the IEEE rule the outputs use. */
uint16_t o_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* ---------------------------------------------------------- q4 format */

static inline int zero_of(const uint32_t *Z, int64_t n, int64_t G, int64_t g) {
    if (!Z) return 8;
    const int64_t zw = (G + 7) / 8;
    return (int)((Z[n * zw + g / 8] >> (4 * (g % 8))) & 0xfu);
}

/* Nibble values q in [0,15], row-major [N][K]. docs/MODEL.md:34-37. */
void o_q4_unpack(const uint32_t *W, int64_t N, int64_t K, uint8_t *out) {
    for (int64_t n = 0; n < N; ++n)
        for (int64_t c = 0; c < K / 8; ++c) {
            const uint32_t word = W[n * (K / 8) + c];
            for (int i = 0; i < 8; ++i) out[n * K + c * 8 + i] = (uint8_t)((word >> (4 * i)) & 0xfu);
        }
}

/* One dequantised row: row[8c+i] = float(q - z) * f16(s), the line
 * ref_model.cpp:114 with the scale read as fp16 and z in place of 8. */
static void dequant_row(const uint32_t *W, const uint16_t *S, const uint32_t *Z, int64_t n, int64_t K, float *row) {
    const int64_t G = K / QGROUP;
    const uint32_t *p = W + n * (K / 8);
    for (int64_t c = 0; c < K / 8; ++c) {
        const int64_t g = c * 8 / QGROUP;
        const float sc = o_f16_to_f32(S[n * G + g]);
        const int z = zero_of(Z, n, G, g);
        const uint32_t word = p[c];
        for (int i = 0; i < 8; ++i) row[c * 8 + i] = (float)((int)((word >> (4 * i)) & 0xfu) - z) * sc;
    }
}

void o_q4_dequant(const uint32_t *W, const uint16_t *S, const uint32_t *Z, int64_t N, int64_t K, float *out) {
    for (int64_t n = 0; n < N; ++n) dequant_row(W, S, Z, n, K, out + n * K);
}

/* ------------------------------------------------------- parallel_for */

/* src/core/threadpool.hpp:38-58: [0,n) split into at most 4*threads chunks of
 * at least `grain` items, handed out dynamically. */
typedef void (*range_fn)(void *ctx, int64_t b, int64_t e);
typedef struct {
    range_fn fn;
    void *ctx;
    int64_t n, chunk, chunks;
    int64_t next; /* atomic */
} pf_job;

static void *pf_worker(void *arg) {
    pf_job *j = (pf_job *)arg;
    for (;;) {
        const int64_t c = __atomic_fetch_add(&j->next, 1, __ATOMIC_RELAXED);
        if (c >= j->chunks) break;
        const int64_t b = c * j->chunk, e = b + j->chunk < j->n ? b + j->chunk : j->n;
        if (b < e) j->fn(j->ctx, b, e);
    }
    return NULL;
}

static void parallel_for(int threads, int64_t n, int64_t grain, range_fn fn, void *ctx) {
    if (n <= 0) return;
    if (grain < 1) grain = 1;
    if (threads < 1) threads = 1;
    int64_t chunks = (n + grain - 1) / grain;
    if (chunks > (int64_t)threads * 4) chunks = (int64_t)threads * 4;
    if (chunks <= 1 || threads == 1) {
        fn(ctx, 0, n);
        return;
    }
    pf_job j = {fn, ctx, n, (n + chunks - 1) / chunks, chunks, 0};
    pthread_t *tids = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int t = 1; t < threads; ++t) pthread_create(&tids[t], NULL, pf_worker, &j);
    pf_worker(&j);
    for (int t = 1; t < threads; ++t) pthread_join(tids[t], NULL);
    free(tids);
}

/* ------------------------------------------------------- expert_linear */

/* ref_model.cpp:25-30 sums a[i]*b[i] in fp32 under `omp simd reduction`,
 * whose order is the compiler's. This restatement fixes one such order:
 * 16 interleaved partial sums, then a pairwise fold. */
static float dot_f32(const float *a, const float *b, int64_t n) {
    float part[16] = {0};
    int64_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 16; ++l) part[l] += a[i + l] * b[i + l];
    for (; i < n; ++i) part[i % 16] += a[i] * b[i];
    for (int w = 8; w > 0; w >>= 1)
        for (int l = 0; l < w; ++l) part[l] += part[l + w];
    return part[0];
}

typedef struct {
    const uint32_t *W;
    const uint16_t *S;
    const uint32_t *Z;
    int64_t K;
    const float *x;
    int T, ldx;
    float *y;
    int ldy;
    double *yd;
} lin_ctx;

static void lin_range(void *vc, int64_t b, int64_t e) {
    lin_ctx *c = (lin_ctx *)vc;
    float *row = (float *)malloc(sizeof(float) * (size_t)c->K);
    for (int64_t o = b; o < e; ++o) {
        dequant_row(c->W, c->S, c->Z, o, c->K, row);
        for (int t = 0; t < c->T; ++t) c->y[(size_t)t * c->ldy + o] = dot_f32(row, c->x + (size_t)t * c->ldx, c->K);
    }
    free(row);
}

/* y[t][o] = sum_i deq(W)[o][i] * x[t][i], the loop of ref_model.cpp:100-119:
 * one dequantised row at a time, dotted against every token, rows split by
 * parallel_for(out, grain 16). */
void o_q4_linear(const uint32_t *W, const uint16_t *S, const uint32_t *Z, int64_t N, int64_t K, const float *x, int T,
                 int ldx, float *y, int ldy, int threads) {
    lin_ctx c = {W, S, Z, K, x, T, ldx, y, ldy, NULL};
    parallel_for(threads, N, 16, lin_range, &c);
}

static void lin_range_f64(void *vc, int64_t b, int64_t e) {
    lin_ctx *c = (lin_ctx *)vc;
    float *row = (float *)malloc(sizeof(float) * (size_t)c->K);
    for (int64_t o = b; o < e; ++o) {
        dequant_row(c->W, c->S, c->Z, o, c->K, row);
        for (int t = 0; t < c->T; ++t) {
            double s = 0.0;
            const float *xt = c->x + (size_t)t * c->ldx;
            for (int64_t i = 0; i < c->K; ++i) s += (double)row[i] * (double)xt[i];
            c->yd[(size_t)t * c->ldy + o] = s;
        }
    }
    free(row);
}

/* The same product as an fp64 brute-force dot on the exact fp32 weights (the
 * method of tests/gpu/test_gemv.hip:57-65): a second, independent answer. */
void o_q4_linear_f64(const uint32_t *W, const uint16_t *S, const uint32_t *Z, int64_t N, int64_t K, const float *x,
                     int T, int ldx, double *y, int ldy, int threads) {
    lin_ctx c = {W, S, Z, K, x, T, ldx, NULL, ldy, y};
    parallel_for(threads, N, 16, lin_range_f64, &c);
}

/* ------------------------------------------------ weight conversion */

/* weight_convert.cpp:61-71: checkpoint order (element 8c+i at bits 4i) to the
 * reference engine's order (even elements in the low half-word, odd ones in
 * the high half-word). */
void o_pack_engine_order(const uint32_t *ct, uint32_t *out, int64_t n_words) {
    for (int64_t i = 0; i < n_words; ++i) {
        uint32_t w = ct[i], r = 0;
        for (int k = 0; k < 8; ++k) {
            const uint32_t nib = (w >> (4 * k)) & 0xfu;
            const int bit = (k & 1) ? 16 + 4 * (k >> 1) : 4 * (k >> 1);
            r |= nib << bit;
        }
        out[i] = r;
    }
}

/* The inverse: reference engine order back to checkpoint order. */
void o_unpack_engine_order(const uint32_t *eng, uint32_t *out, int64_t n_words) {
    for (int64_t i = 0; i < n_words; ++i) {
        uint32_t w = eng[i], r = 0;
        for (int k = 0; k < 8; ++k) {
            const int bit = (k & 1) ? 16 + 4 * (k >> 1) : 4 * (k >> 1);
            r |= ((w >> bit) & 0xfu) << (4 * k);
        }
        out[i] = r;
    }
}

/* weight_convert.cpp:73-90: symmetric int4 g128 (scale = amax/7 as fp16,
 * q = clamp(lrint(x/scale), -8, 7) + 8), checkpoint word order. */
void o_quantize_g128(const uint16_t *src_bf16, int64_t n_groups, uint32_t *words, uint16_t *scales) {
    for (int64_t g = 0; g < n_groups; ++g) {
        const uint16_t *x = src_bf16 + g * QGROUP;
        float amax = 0.f;
        for (int k = 0; k < QGROUP; ++k) {
            const float a = fabsf(o_bf16_to_f32(x[k]));
            amax = a > amax ? a : amax;
        }
        const uint16_t sc16 = o_f32_to_f16(amax / 7.f);
        const float sc = o_f16_to_f32(sc16), inv = sc > 0.f ? 1.f / sc : 0.f;
        for (int k = 0; k < QGROUP; k += 8) {
            uint32_t word = 0;
            for (int j = 0; j < 8; ++j) {
                long q = lrintf(o_bf16_to_f32(x[k + j]) * inv);
                q = q < -8 ? -8 : (q > 7 ? 7 : q);
                word |= (uint32_t)(q + 8) << (4 * j);
            }
            words[(g * QGROUP + k) / 8] = word;
        }
        scales[g] = sc16;
    }
}

/* ------------------------------------------------------------- routing */

/* ref_model.cpp:412-431 for one token: p = exp(l - max) in fp32, the top k by
 * (p descending, index ascending), weights float(p / sum_top p) with the sum
 * in double in selection order. */
void o_route(const float *logits, int T, int E, int topk, int32_t *top_e, float *top_w) {
    float *pr = (float *)malloc(sizeof(float) * (size_t)E);
    char *used = (char *)malloc((size_t)E);
    for (int t = 0; t < T; ++t) {
        const float *l = logits + (size_t)t * E;
        float mx = l[0];
        for (int e = 1; e < E; ++e) mx = l[e] > mx ? l[e] : mx;
        for (int e = 0; e < E; ++e) pr[e] = expf(l[e] - mx);
        memset(used, 0, (size_t)E);
        /* selection sort of the first k: the same order partial_sort yields
         * under the strict comparator (p desc, index asc). */
        for (int i = 0; i < topk; ++i) {
            int best = -1;
            for (int e = 0; e < E; ++e) {
                if (used[e]) continue;
                if (best < 0 || pr[e] > pr[best]) best = e;
            }
            used[best] = 1;
            top_e[(size_t)t * topk + i] = best;
        }
        double top = 0.0;
        for (int i = 0; i < topk; ++i) top += (double)pr[top_e[(size_t)t * topk + i]];
        for (int i = 0; i < topk; ++i)
            top_w[(size_t)t * topk + i] = (float)((double)pr[top_e[(size_t)t * topk + i]] / top);
    }
    free(used);
    free(pr);
}

/* Gather order of ref_model.cpp:411-431 (by_expert[e] filled in ascending
 * token order) and of moe_route.hip:149-160: experts ascending, pairs of one
 * expert in (token, k) order. counts[E], offsets[E+1], tok_slot[T*k],
 * pair_tok[T*k]. */
void o_moe_slots(const int32_t *top_e, int T, int E, int topk, int32_t *counts, int32_t *offsets, int32_t *tok_slot,
                 int32_t *pair_tok) {
    memset(counts, 0, sizeof(int32_t) * (size_t)E);
    for (int i = 0; i < T * topk; ++i) counts[top_e[i]]++;
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t *fill = (int32_t *)calloc((size_t)E, sizeof(int32_t));
    for (int i = 0; i < T * topk; ++i) {
        const int e = top_e[i];
        const int slot = offsets[e] + fill[e]++;
        tok_slot[i] = slot;
        pair_tok[slot] = i / topk;
    }
    free(fill);
}

static float o_silu(float x) { return x * (1.f / (1.f + expf(-x))); }

/* ref_model.cpp:406-463 (the routed experts; the shared expert is
 * o_linear_w16 + o_swiglu_gate below, composed in oracle.py's
 * shared_expert): route, then for each expert in ascending order gather its tokens,
 * g = gate x, u = up x, h = silu(g) u, y = down h, out[t] += w y.
 * Weights per expert are contiguous: gate/up [E][F][H/8], down [E][H][F/8].
 * Also returns h [T*k][F] and yp [T*k][H] in slot order when non-NULL. */
void o_moe(const float *x, int T, int H, int F, int E, int topk, const float *logits, const uint32_t *gw,
           const uint16_t *gs, const uint32_t *gz, const uint32_t *uw, const uint16_t *us, const uint32_t *uz,
           const uint32_t *dw, const uint16_t *ds, const uint32_t *dz, float *out, float *h_out, float *yp_out,
           int threads) {
    const int P = T * topk;
    int32_t *top_e = (int32_t *)malloc(sizeof(int32_t) * (size_t)P);
    float *top_w = (float *)malloc(sizeof(float) * (size_t)P);
    int32_t *counts = (int32_t *)malloc(sizeof(int32_t) * (size_t)E);
    int32_t *offsets = (int32_t *)malloc(sizeof(int32_t) * (size_t)(E + 1));
    int32_t *tok_slot = (int32_t *)malloc(sizeof(int32_t) * (size_t)P);
    int32_t *pair_tok = (int32_t *)malloc(sizeof(int32_t) * (size_t)P);
    o_route(logits, T, E, topk, top_e, top_w);
    o_moe_slots(top_e, T, E, topk, counts, offsets, tok_slot, pair_tok);
    float *slot_w = (float *)malloc(sizeof(float) * (size_t)P);
    for (int i = 0; i < P; ++i) slot_w[tok_slot[i]] = top_w[i];

    const int GH = H / QGROUP, GF = F / QGROUP;
    const int zwH = (GH + 7) / 8, zwF = (GF + 7) / 8;
    memset(out, 0, sizeof(float) * (size_t)T * (size_t)H);
    float *xs = (float *)malloc(sizeof(float) * (size_t)T * (size_t)H);
    float *g = (float *)malloc(sizeof(float) * (size_t)T * (size_t)F);
    float *u = (float *)malloc(sizeof(float) * (size_t)T * (size_t)F);
    float *y = (float *)malloc(sizeof(float) * (size_t)T * (size_t)H);
    for (int e = 0; e < E; ++e) {
        const int n = counts[e];
        if (!n) continue;
        const int base = offsets[e];
        for (int i = 0; i < n; ++i) memcpy(xs + (size_t)i * H, x + (size_t)pair_tok[base + i] * H, sizeof(float) * (size_t)H);
        const size_t guw = (size_t)e * F * (H / 8), gus = (size_t)e * F * GH, guz = (size_t)e * F * zwH;
        o_q4_linear(gw + guw, gs + gus, gz ? gz + guz : NULL, F, H, xs, n, H, g, F, threads);
        o_q4_linear(uw + guw, us + gus, uz ? uz + guz : NULL, F, H, xs, n, H, u, F, threads);
        for (size_t i = 0; i < (size_t)n * F; ++i) g[i] = o_silu(g[i]) * u[i];
        const size_t dww = (size_t)e * H * (F / 8), dss = (size_t)e * H * GF, dzz = (size_t)e * H * zwF;
        o_q4_linear(dw + dww, ds + dss, dz ? dz + dzz : NULL, H, F, g, n, F, y, H, threads);
        if (h_out) memcpy(h_out + (size_t)base * F, g, sizeof(float) * (size_t)n * F);
        if (yp_out) memcpy(yp_out + (size_t)base * H, y, sizeof(float) * (size_t)n * H);
        for (int i = 0; i < n; ++i) {
            const float w = slot_w[base + i];
            float *o = out + (size_t)pair_tok[base + i] * H;
            for (int j = 0; j < H; ++j) o[j] += w * y[(size_t)i * H + j];
        }
    }
    free(xs);
    free(g);
    free(u);
    free(y);
    free(slot_w);
    free(top_e);
    free(top_w);
    free(counts);
    free(offsets);
    free(tok_slot);
    free(pair_tok);
}

/* ---------------------------------------------- 16-bit dense weights */

typedef struct {
    const uint16_t *W;
    int f16;
    int64_t K, ldw;
    const float *x;
    int T, ldx;
    float *y;
    int ldy;
} lin16_ctx;

static void lin16_range(void *vc, int64_t b, int64_t e) {
    lin16_ctx *c = (lin16_ctx *)vc;
    float *row = (float *)malloc(sizeof(float) * (size_t)c->K);
    for (int64_t o = b; o < e; ++o) {
        const uint16_t *w = c->W + (size_t)o * (size_t)c->ldw;
        for (int64_t i = 0; i < c->K; ++i) row[i] = c->f16 ? o_f16_to_f32(w[i]) : o_bf16_to_f32(w[i]);
        for (int t = 0; t < c->T; ++t) c->y[(size_t)t * c->ldy + o] = dot_f32(row, c->x + (size_t)t * c->ldx, c->K);
    }
    free(row);
}

/* ref::Model::linear (src/ref/ref_model.cpp:86-97): y[t][o] = sum_i W[o][i] x[t][i]
 * with W 16-bit (bf16 there; fp16 as in gpu::gemv_rows, src/kernels/gemv.hip:7-42,
 * when f16 != 0), each row widened to fp32 and dotted in fp32. */
void o_linear_w16(const uint16_t *W, int f16, int64_t N, int64_t K, int64_t ldw, const float *x, int T, int ldx,
                  float *y, int ldy, int threads) {
    lin16_ctx c = {W, f16, K, ldw, x, T, ldx, y, ldy};
    parallel_for(threads, N, 16, lin16_range, &c);
}

/* weight_convert.cpp:92-108 (quantize_rows_i8): per row and group of `group`
 * weights along K, s = amax / 127 over the group's fp16 weights widened to
 * fp32 (1 when amax is 0), q = lrint(clamp(w / s, -127, 127)) (round to
 * nearest even, the default rounding mode). */
void o_quantize_rows_i8(const uint16_t *w16, int64_t N, int64_t K, int64_t group, int8_t *q, float *scale) {
    const int64_t G = K / group;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t g = 0; g < G; ++g) {
            const uint16_t *w = w16 + n * K + g * group;
            float amax = 0.f;
            for (int64_t k = 0; k < group; ++k) amax = fmaxf(amax, fabsf(o_f16_to_f32(w[k])));
            const float s = amax > 0.f ? amax / 127.f : 1.f;
            scale[n * G + g] = s;
            for (int64_t k = 0; k < group; ++k) {
                float v = o_f16_to_f32(w[k]) / s;
                v = v < -127.f ? -127.f : v > 127.f ? 127.f : v;
                q[n * K + g * group + k] = (int8_t)lrintf(v);
            }
        }
}

typedef struct {
    const int8_t *W8;
    const float *scale;
    int64_t K;
    int group;
    const uint16_t *x;
    int xs, M, rpg;
    double *y;
    int ys;
} i8_ctx;

static void i8_range(void *vc, int64_t b, int64_t e) {
    i8_ctx *c = (i8_ctx *)vc;
    const int64_t G = c->K / c->group;
    for (int64_t n = b; n < e; ++n) {
        const int8_t *w = c->W8 + n * c->K;
        const float *s = c->scale + n * G;
        const int64_t off = c->rpg > 0 ? (n / c->rpg) * c->K : 0;
        for (int m = 0; m < c->M; ++m) {
            const uint16_t *x = c->x + (int64_t)m * c->xs + off;
            double acc = 0.0;
            for (int64_t k = 0; k < c->K; ++k) acc += (double)w[k] * (double)s[k / c->group] * (double)o_f16_to_f32(x[k]);
            c->y[(int64_t)m * c->ys + n] = acc;
        }
    }
}

/* gpu::gemv_rows_i8 (src/kernels/gemv.hip:75-136, declared gemv.hpp:15-23):
 *   y[m*ys + n] = sum_k W8[n][k] * scale[n][k / group] * x[m*xs + off(n) + k]
 * with off(n) = (n / rpg) * K for rpg > 0 (rows grouped over activation
 * blocks), x fp16 bits; the sum in fp64, as the reference's own test forms
 * its expected values (tests/gpu/test_gemv.hip:93-104). */
void o_i8_linear_f64(const int8_t *W8, const float *scale, int64_t N, int64_t K, int group, const uint16_t *x, int xs,
                     int M, int rpg, double *y, int ys, int threads) {
    i8_ctx c = {W8, scale, K, group, x, xs, M, rpg, y, ys};
    parallel_for(threads, N, 16, i8_range, &c);
}

static float o_sigmoid(float x) { return 1.f / (1.f + expf(-x)); }

/* The shared expert's activation (ref_model.cpp:468-476 with the gate folded
 * in, the role of gpu::swiglu_T, src/kernels/moe_route.hip:187-197):
 *   h[t][j] = silu(v[t][j]) * v[t][n + j] * sigmoid(v[t][2n])
 * for v [T][ldv] holding gate (n), up (n) and the gate logit (1) per row. */
void o_swiglu_gate(const float *v, int ldv, int n, int T, float *h) {
    for (int t = 0; t < T; ++t) {
        const float *r = v + (size_t)t * ldv;
        const float gsig = o_sigmoid(r[2 * n]);
        for (int j = 0; j < n; ++j) h[(size_t)t * n + j] = o_silu(r[j]) * r[n + j] * gsig;
    }
}

/* ------------------------------------------------- device tiled format */

/* The kernels' weight layout (this build's load-time repack, the role of
 * pack_int4_words in src/engine/weight_convert.cpp:61-71):
 *   Wt  uint4 [N/16][G][4][16]: entry (sub, g, q, n) = the 16 bytes of row
 *       16*sub+n covering words g*16+4q .. g*16+4q+3, each word with its
 *       nibbles reordered so that element j (j < 4) sits at bits 8j and
 *       element j+4 at bits 8j+4;
 *   St  fp16  [N/16][ceil(G/4)][16][4]: St[sub][gc][n][j] = S[16 sub+n][4 gc+j]
 *       (0 past G);
 *   Zt  u16   [N/16][ceil(G/4)][16]: nibble j = zero of group 4 gc+j (0 past G).
 * N must be a multiple of 16. */
static uint32_t shuffle_word(uint32_t w) {
    uint32_t r = 0;
    for (int j = 0; j < 4; ++j) {
        r |= ((w >> (4 * j)) & 0xfu) << (8 * j);
        r |= ((w >> (4 * (j + 4))) & 0xfu) << (8 * j + 4);
    }
    return r;
}

void o_q4_tile(const uint32_t *W, const uint16_t *S, const uint32_t *Z, int64_t N, int64_t K, uint32_t *Wt, uint16_t *St,
               uint16_t *Zt) {
    const int64_t G = K / QGROUP, GC = (G + 3) / 4, subs = N / 16;
    for (int64_t sub = 0; sub < subs; ++sub)
        for (int64_t g = 0; g < G; ++g)
            for (int q = 0; q < 4; ++q)
                for (int n = 0; n < 16; ++n)
                    for (int j = 0; j < 4; ++j) {
                        const int64_t row = sub * 16 + n;
                        Wt[(((sub * G + g) * 4 + q) * 16 + n) * 4 + j] = shuffle_word(W[row * (K / 8) + g * 16 + q * 4 + j]);
                    }
    for (int64_t sub = 0; sub < subs; ++sub)
        for (int64_t gc = 0; gc < GC; ++gc)
            for (int n = 0; n < 16; ++n) {
                const int64_t row = sub * 16 + n;
                uint16_t zt = 0;
                for (int j = 0; j < 4; ++j) {
                    const int64_t g = gc * 4 + j;
                    St[((sub * GC + gc) * 16 + n) * 4 + j] = g < G ? S[row * G + g] : 0;
                    if (g < G && Z) zt |= (uint16_t)(zero_of(Z, row, G, g) << (4 * j));
                }
                if (Zt) Zt[(sub * GC + gc) * 16 + n] = zt;
            }
}

/* ----------------------------------------------------------------- W4A8 */

/* gpu::moe_experts_w4a8's activation quantiser, quant_rows_kernel
 * (src/kernels/moe_w4a8.hip:17-36): per row and group of 128 along K,
 * sc = max|x| / 127 (1 when the group is all zero), inv = 1 / sc (fp32
 * division), q = int8(rint(x * inv)) (round half to even; |x * inv| <= 127
 * up to an ulp, so no clamp is needed). x holds 16-bit bits: fp16 when
 * f16 != 0 (the reference's rows), else bf16. */
void o_quant_rows_i8(const uint16_t *x, int f16, int64_t rows, int64_t K, int64_t ldx, int8_t *q, float *scale) {
    const int64_t G = K / QGROUP;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t g = 0; g < G; ++g) {
            const uint16_t *xg = x + r * ldx + g * QGROUP;
            float v[QGROUP], mx = 0.f;
            for (int i = 0; i < QGROUP; ++i) {
                v[i] = f16 ? o_f16_to_f32(xg[i]) : o_bf16_to_f32(xg[i]);
                mx = fmaxf(mx, fabsf(v[i]));
            }
            const float sc = mx > 0.f ? mx / 127.f : 1.f, inv = 1.f / sc;
            for (int i = 0; i < QGROUP; ++i) q[r * K + g * QGROUP + i] = (int8_t)(int)rintf(v[i] * inv);
            scale[r * G + g] = sc;
        }
}

typedef struct {
    const int8_t *q8;
    const float *sx;
    const int32_t *rowmap;
    int64_t K;
    const uint32_t *W;
    const uint16_t *S;
    const uint32_t *Z;
    int64_t N;
    float *y;
} w4a8_ctx;

static void w4a8_range(void *vc, int64_t b, int64_t e) {
    const w4a8_ctx *c = (const w4a8_ctx *)vc;
    const int64_t K = c->K, G = K / QGROUP;
    int8_t *wq = (int8_t *)malloc((size_t)K);
    for (int64_t n = 0; n < c->N; ++n) {
        /* the row widened exactly: q - z (moe_w4a8.hip:38-56 with z = 8) */
        for (int64_t k = 0; k < K; ++k) {
            const uint32_t word = c->W[n * (K / 8) + k / 8];
            wq[k] = (int8_t)((int)((word >> (4 * (k % 8))) & 0xfu) - zero_of(c->Z, n, G, k / QGROUP));
        }
        for (int64_t p = b; p < e; ++p) {
            const int64_t r = c->rowmap ? c->rowmap[p] : p;
            const int8_t *a = c->q8 + r * K;
            float acc = 0.f;
            /* int32 per 64-wide K step, then the step's group scales in
             * fp32, steps in order: acc += float(dot) * s_w * s_x, the
             * last multiply-add fused as the HIP compiler contracts it
             * (moe_w4a8.hip:98-116, :161-176) */
            for (int64_t k0 = 0; k0 < K; k0 += 64) {
                int32_t dot = 0;
                for (int k = 0; k < 64; ++k) dot += (int32_t)a[k0 + k] * (int32_t)wq[k0 + k];
                const int64_t g = k0 / QGROUP;
                const float sw = o_f16_to_f32(c->S[n * G + g]);
                acc = fmaf((float)dot * sw, c->sx[r * G + g], acc);
            }
            c->y[p * c->N + n] = acc;
        }
    }
    free(wq);
}

/* One W4A8 projection of the grouped expert GEMMs (moe_w4a8.hip:62-118,
 * :120-183): for P activation rows (row p of the product reads quantised row
 * rowmap[p], or p when rowmap is NULL: the gathered token of a slot for
 * gate / up, the slot itself for down) and N weight rows,
 *   y[p][n] = sum over 64-wide K steps, in order, of float(I) * s_w * s_x
 * with I the exact int32 dot of the step. q8 / sx as o_quant_rows_i8 writes
 * them (row stride K); W, S, Z in this build's checkpoint formats. */
void o_w4a8_linear(const int8_t *q8, const float *sx, const int32_t *rowmap, int64_t P, int64_t K, const uint32_t *W,
                   const uint16_t *S, const uint32_t *Z, int64_t N, float *y, int threads) {
    w4a8_ctx c = {q8, sx, rowmap, K, W, S, Z, N, y};
    parallel_for(threads, P, 4, w4a8_range, &c);
}
