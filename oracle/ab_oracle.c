/*
 * CPU oracle for the AB-Attention selection and weighted paged prefill.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker for the HIP library:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it. Nothing in the product path links or calls it.
 *
 * Each function restates the reference algorithm (paths relative to the
 * reference checkout) with the association order of every floating-point
 * sum written out explicitly:
 *
 *   orc_cluster   csrc/ibcs.cu:106-238 (+ the centroid scaling at :293-295)
 *   orc_pool      csrc/ibcs.cu:244-266
 *   orc_lse       csrc/ibcs.cu:329-368, :370-489
 *   orc_masses    csrc/ibcs.cu:495-538
 *   orc_sip       csrc/sip.cu:33-167
 *   orc_prefill   ab_attention/flashinfer_backend.py:30-59, :164-242
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp). Contraction
 * is off so that every fused multiply-add below is one the restatement asks
 * for with fmaf()/fma(), mirroring where nvcc's default contraction fuses
 * `a += b * c` in the reference build.
 *
 * Rows (query blocks) are independent in every stage, so the row loops run
 * in parallel over OpenMP threads; each row is computed by one thread in the
 * order written here, so the results do not depend on the thread count.
 *
 * Deliberate restatement choices (the reference build uses --use_fast_math,
 * whose approximate division/exp2/log2 are not reproduced):
 *   - float division is IEEE division;
 *   - exp2f/log2f are the C library's;
 *   - in orc_masses the per-centroid division by the normaliser is a
 *     multiplication by its reciprocal, computed once per (row, centroid).
 */
#include <float.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define HEAD_DIM 128
#define QUERY_BLOCK 128
#define CENTROIDS 8
#define KV_BLOCK 4
#define REPS 2
#define SIP_THREADS 256
#define SIP_WARP 32
#define SIP_BUCKET 4

/* ---- number formats ------------------------------------------------------ */

static inline float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Round-to-nearest-even float -> bfloat16 (NaN kept quiet). */
static inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* Round-to-nearest-even float -> IEEE binary16, including subnormals. */
static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                   /* below 2^-14: subnormal */
        float af;
        memcpy(&af, &ax, 4);
        const uint32_t m = (uint32_t)nearbyintf(af * 16777216.0f); /* exact scale by 2^24 */
        return (uint16_t)(sign | m);
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

static float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    float f;
    if (e == 0) {
        f = ldexpf((float)m, -24);
        return sign ? -f : f;
    }
    uint32_t u = (e == 31) ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
    memcpy(&f, &u, 4);
    return f;
}

/* Exported for the tests' format checks. */
uint16_t orc_f32_to_f16(float f) { return f32_to_f16(f); }
float orc_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t orc_f32_to_bf16(float f) { return f32_to_bf16(f); }

/* Threads the parallel row loops use (OMP_NUM_THREADS, else all host threads). */
int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---- IBCS stage 1: query clustering (csrc/ibcs.cu:106-238) -------------- */

/*
 * Squared distance with the reference's association: lane l (0..31) chains
 * fmaf over dims l, l+32, l+64, l+96 (ibcs.cu:143-150, :173-180), then an
 * xor butterfly with masks 16,8,4,2,1 (warp_sum, ibcs.cu:61-67). Every lane
 * of a butterfly ends with the same value, equal to the pairwise tree below.
 */
static float lane_distance(const float *a, const float *b) {
    float p[32];
    for (int lane = 0; lane < 32; ++lane) {
        float acc = 0.0f;
        for (int d = lane; d < HEAD_DIM; d += 32) {
            const float delta = a[d] - b[d];
            acc = fmaf(delta, delta, acc);
        }
        p[lane] = acc;
    }
    for (int mask = 16; mask >= 1; mask >>= 1)
        for (int lane = 0; lane < mask; ++lane) p[lane] = p[lane] + p[lane + mask];
    return p[0];
}

/* cub::ArgMax over one value per thread: largest value, lowest index on ties
 * (ibcs.cu:94-102). Threads at or beyond `valid` contribute -inf. */
static int argmax_lowest(const float *v, int valid) {
    int best = 0;
    float bv = valid > 0 ? v[0] : -INFINITY;
    for (int i = 1; i < valid; ++i)
        if (v[i] > bv) {
            bv = v[i];
            best = i;
        }
    return best;
}

/*
 * q: bf16 [bh, n, 128]. Outputs per row (bh * qb + block):
 *   centroids: bf16 [rows, 8, 128], already scaled: bf16(float(bf16(mean)) * scale)
 *              (the scaling is load_q_centroid_pair, ibcs.cu:293-295);
 *   pops:      float [rows, 8] cluster populations (the reference stores them
 *              as fp16, exact for counts <= 128).
 */
void orc_cluster(const uint16_t *q, int64_t bh_count, int64_t n, float qk_scale_log2,
                 uint16_t *centroids, float *pops) {
    const int64_t qb = (n + QUERY_BLOCK - 1) / QUERY_BLOCK;
#pragma omp parallel for schedule(dynamic, 8)
    for (int64_t row_index = 0; row_index < bh_count * qb; ++row_index) {
        const int64_t bh = row_index / qb, blk = row_index % qb;
        float x[QUERY_BLOCK][HEAD_DIM];
        float mean[HEAD_DIM], min_d[QUERY_BLOCK];
        int assign[QUERY_BLOCK];
        const int64_t base = blk * QUERY_BLOCK;
        const int valid = (int)((n - base) < QUERY_BLOCK ? (n - base) : QUERY_BLOCK);
        for (int i = 0; i < valid; ++i)
            for (int d = 0; d < HEAD_DIM; ++d)
                x[i][d] = bf16_to_f32(q[((bh * n) + base + i) * HEAD_DIM + d]);
        for (int d = 0; d < HEAD_DIM; ++d) {
            float sum = 0.0f;
            for (int i = 0; i < valid; ++i) sum += x[i][d];
            mean[d] = sum / (float)valid;
        }
        for (int i = 0; i < valid; ++i) min_d[i] = lane_distance(x[i], mean);
        int center = argmax_lowest(min_d, valid);
        for (int i = 0; i < valid; ++i) {
            min_d[i] = INFINITY;
            assign[i] = 0;
        }
        for (int slot = 0; slot < CENTROIDS; ++slot) {
            for (int i = 0; i < valid; ++i) {
                const float dist = lane_distance(x[i], x[center]);
                if (dist < min_d[i]) {
                    min_d[i] = dist;
                    assign[i] = slot;
                }
            }
            if (slot + 1 < CENTROIDS) center = argmax_lowest(min_d, valid);
        }
        int counts[CENTROIDS] = {0};
        for (int i = 0; i < valid; ++i) ++counts[assign[i]];
        const int64_t row = bh * qb + blk;
        for (int s = 0; s < CENTROIDS; ++s) pops[row * CENTROIDS + s] = (float)counts[s];
        for (int d = 0; d < HEAD_DIM; ++d) {
            float sums[CENTROIDS] = {0};
            for (int i = 0; i < valid; ++i) sums[assign[i]] += x[i][d];
            for (int s = 0; s < CENTROIDS; ++s) {
                const uint16_t c = counts[s] > 0 ? f32_to_bf16(sums[s] / (float)counts[s])
                                                 : f32_to_bf16(0.0f);
                centroids[(row * CENTROIDS + s) * HEAD_DIM + d] =
                    f32_to_bf16(bf16_to_f32(c) * qk_scale_log2);
            }
        }
    }
}

/* ---- IBCS stage 2: key pooling (csrc/ibcs.cu:244-266) ------------------- */

/* k: bf16 [bh, n, 128] -> pooled bf16 [bh, n/4, 2, 128]. */
void orc_pool(const uint16_t *k, int64_t bh_count, int64_t n, uint16_t *pooled) {
    const int64_t fb = n / KV_BLOCK;
#pragma omp parallel for schedule(static)
    for (int64_t bh = 0; bh < bh_count; ++bh)
        for (int64_t j = 0; j < fb; ++j)
            for (int r = 0; r < REPS; ++r)
                for (int d = 0; d < HEAD_DIM; ++d) {
                    const int64_t t0 = (bh * n + KV_BLOCK * j + 2 * r) * HEAD_DIM + d;
                    const float value = 0.5f * (bf16_to_f32(k[t0]) + bf16_to_f32(k[t0 + HEAD_DIM]));
                    pooled[((bh * fb + j) * REPS + r) * HEAD_DIM + d] = f32_to_bf16(value);
                }
}

/* ---- IBCS stage 3: centroid/key LSE (csrc/ibcs.cu:329-489) ------------- */

/* pair_lse (ibcs.cu:339-343). */
static float pair_lse(float left, float right) {
    const float maximum = fmaxf(left, right);
    return maximum + log2f(fmaxf(exp2f(left - maximum) + exp2f(right - maximum), 1.0e-20f));
}

/* accumulate_lse (ibcs.cu:329-335); nvcc fuses the first product. */
static void accumulate_lse(float *maximum, float *den, float value) {
    const float next = fmaxf(*maximum, value);
    *den = fmaf(*den, exp2f(*maximum - next), exp2f(value - next));
    *maximum = next;
}

/* combine_lse (ibcs.cu:362-368), from the point of view of the lane that
 * keeps the result. */
static void combine_lse(float *maximum, float *den, float other_max, float other_den) {
    const float next = fmaxf(*maximum, other_max);
    *den = fmaf(*den, exp2f(*maximum - next), other_den * exp2f(other_max - next));
    *maximum = next;
}

/*
 * centroids: scaled bf16 [rows, 8, 128]; pooled: bf16 [bh, fb, 2, 128].
 * Outputs: lse fp16 bits [rows, 8, fb]; lse_max, lse_den float [rows, 8].
 *
 * Dot products are exact sums of exact bf16 products rounded once to float
 * (the reference's tensor-core accumulation order is not defined). Each
 * (row, centroid) normaliser follows ibcs.cu:421-477: four lanes own the
 * blocks j = c (mod 4), fold them in ascending order from the fp16-rounded
 * values, then merge with xor masks 1 and 2.
 */
void orc_lse_rows(const uint16_t *centroids, int64_t rows, const uint16_t *pooled, int64_t fb,
                  uint16_t *lse, float *lse_max, float *lse_den) {
    float *rep = (float *)malloc(sizeof(float) * (size_t)fb * REPS * HEAD_DIM);
    if (!rep) return;
    for (int64_t i = 0; i < fb * REPS * HEAD_DIM; ++i) rep[i] = bf16_to_f32(pooled[i]);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t row = 0; row < rows; ++row) {
        for (int s = 0; s < CENTROIDS; ++s) {
            float c[HEAD_DIM];
            for (int d = 0; d < HEAD_DIM; ++d)
                c[d] = bf16_to_f32(centroids[(row * CENTROIDS + s) * HEAD_DIM + d]);
            float lm[4], ld[4];
            for (int l = 0; l < 4; ++l) {
                lm[l] = -FLT_MAX;
                ld[l] = 0.0f;
            }
            uint16_t *out = lse + (row * CENTROIDS + s) * fb;
            for (int64_t j = 0; j < fb; ++j) {
                float t[REPS];
                for (int r = 0; r < REPS; ++r) {
                    const float *kr = rep + (j * REPS + r) * HEAD_DIM;
                    double acc = 0.0;
                    for (int d = 0; d < HEAD_DIM; ++d) acc += (double)c[d] * (double)kr[d];
                    t[r] = (float)acc;
                }
                const uint16_t h = f32_to_f16(pair_lse(t[0] + 1.0f, t[1] + 1.0f));
                out[j] = h;
                accumulate_lse(&lm[j & 3], &ld[j & 3], f16_to_f32(h));
            }
            /* xor 1: lane 0 takes lane 1, lane 2 takes lane 3; xor 2: lane 0 takes lane 2 */
            combine_lse(&lm[0], &ld[0], lm[1], ld[1]);
            combine_lse(&lm[2], &ld[2], lm[3], ld[3]);
            combine_lse(&lm[0], &ld[0], lm[2], ld[2]);
            lse_max[row * CENTROIDS + s] = lm[0];
            lse_den[row * CENTROIDS + s] = ld[0];
        }
    }
    free(rep);
}

/* Every row of every head: rows of head bh are bh*qb .. bh*qb+qb-1. */
void orc_lse(const uint16_t *centroids, const uint16_t *pooled, int64_t bh_count, int64_t n,
             uint16_t *lse, float *lse_max, float *lse_den) {
    const int64_t qb = (n + QUERY_BLOCK - 1) / QUERY_BLOCK;
    const int64_t fb = n / KV_BLOCK;
    for (int64_t bh = 0; bh < bh_count; ++bh) {
        const int64_t row0 = bh * qb;
        orc_lse_rows(centroids + row0 * CENTROIDS * HEAD_DIM, qb, pooled + bh * fb * REPS * HEAD_DIM, fb,
                     lse + row0 * CENTROIDS * fb, lse_max + row0 * CENTROIDS, lse_den + row0 * CENTROIDS);
    }
}

/* ---- IBCS stage 4: population-weighted masses (csrc/ibcs.cu:495-538) ---- */

/* m_j = (sum_s fmaf(n_s, exp2f(l_sj - M_s) * (1/D_s), .)) * (1/sum_s n_s). */
void orc_masses(const uint16_t *lse, const float *pops, const float *lse_max, const float *lse_den,
                int64_t rows, int64_t fb, float *scores) {
#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t row = 0; row < rows; ++row) {
        float weight[CENTROIDS], inv_den[CENTROIDS], mx[CENTROIDS];
        float total = 0.0f;
        for (int s = 0; s < CENTROIDS; ++s) {
            weight[s] = pops[row * CENTROIDS + s];
            inv_den[s] = 1.0f / lse_den[row * CENTROIDS + s];
            mx[s] = lse_max[row * CENTROIDS + s];
            total += weight[s];
        }
        const float inv_total = 1.0f / total;
        for (int64_t j = 0; j < fb; ++j) {
            float score = 0.0f;
            for (int s = 0; s < CENTROIDS; ++s) {
                const float value = f16_to_f32(lse[(row * CENTROIDS + s) * fb + j]);
                score = fmaf(weight[s], exp2f(value - mx[s]) * inv_den[s], score);
            }
            scores[row * fb + j] = score * inv_total;
        }
    }
}

/* Whole IBCS for bf16 q/k [bh, n, 128] -> scores [bh*qb, n/4]. */
int orc_ibcs(const uint16_t *q, const uint16_t *k, int64_t bh_count, int64_t n, float qk_scale_log2,
             float *scores) {
    const int64_t qb = (n + QUERY_BLOCK - 1) / QUERY_BLOCK, fb = n / KV_BLOCK, rows = bh_count * qb;
    uint16_t *cent = malloc(sizeof(uint16_t) * (size_t)rows * CENTROIDS * HEAD_DIM);
    float *pops = malloc(sizeof(float) * (size_t)rows * CENTROIDS);
    uint16_t *pooled = malloc(sizeof(uint16_t) * (size_t)bh_count * fb * REPS * HEAD_DIM);
    uint16_t *lse = malloc(sizeof(uint16_t) * (size_t)rows * CENTROIDS * fb);
    float *mx = malloc(sizeof(float) * (size_t)rows * CENTROIDS);
    float *den = malloc(sizeof(float) * (size_t)rows * CENTROIDS);
    int rc = (cent && pops && pooled && lse && mx && den) ? 0 : 1;
    if (!rc) {
        orc_cluster(q, bh_count, n, qk_scale_log2, cent, pops);
        orc_pool(k, bh_count, n, pooled);
        orc_lse(cent, pooled, bh_count, n, lse, mx, den);
        orc_masses(lse, pops, mx, den, rows, fb, scores);
    }
    free(cent);
    free(pops);
    free(pooled);
    free(lse);
    free(mx);
    free(den);
    return rc;
}

/* ---- SIP (csrc/sip.cu:33-167) ------------------------------------------- */

/*
 * cub::BlockReduce<.., 256> (BLOCK_REDUCE_WARP_REDUCTIONS) of one double per
 * thread: each 32-thread warp reduces with shfl_down offsets 1,2,4,8,16
 * (lane i adds lane i+o), giving the pairwise tree below; thread 0 then folds
 * the eight warp totals left to right.
 */
static double block_sum(const double *part) {
    double total = 0.0;
    for (int w = 0; w < SIP_THREADS / SIP_WARP; ++w) {
        double t[SIP_WARP];
        memcpy(t, part + w * SIP_WARP, sizeof(t));
        for (int off = 1; off < SIP_WARP; off <<= 1)
            for (int i = 0; i + off < SIP_WARP; i += 2 * off) t[i] = t[i] + t[i + off];
        total = (w == 0) ? t[0] : total + t[0];
    }
    return total;
}

/*
 * cub::BlockScan<double, 256>::ExclusiveSum (BLOCK_SCAN_RAKING): 32 raking
 * threads each fold 8 consecutive partials left to right, a 32-lane
 * Kogge-Stone inclusive scan (shfl_up 1,2,4,8,16), shift by one lane
 * (lane 0 gets 0.0), then each segment is rescanned from its prefix.
 */
static void block_exclusive_sum(const double *in, double *out) {
    double raking[32], inc[32];
    for (int r = 0; r < 32; ++r) {
        double acc = in[8 * r];
        for (int i = 1; i < 8; ++i) acc = acc + in[8 * r + i];
        raking[r] = acc;
    }
    memcpy(inc, raking, sizeof(inc));
    for (int off = 1; off < 32; off <<= 1) {
        double next[32];
        for (int r = 0; r < 32; ++r) next[r] = (r >= off) ? inc[r - off] + inc[r] : inc[r];
        memcpy(inc, next, sizeof(inc));
    }
    for (int r = 0; r < 32; ++r) {
        double ex = (r == 0) ? 0.0 : 0.0 + inc[r - 1];
        for (int i = 0; i < 8; ++i) {
            out[8 * r + i] = ex;
            ex = ex + in[8 * r + i];
        }
    }
}

/* One row of SIP: input [pop] masses, offset_f its uniform -> out/logs
 * [samples]; values [pop] and prefix [buckets + 1] are scratch. */
static void sip_row(const float *input, float offset_f, int pop, int64_t samples, int32_t *out, float *logs,
                    float *values, double *prefix) {
    const int buckets = (pop + SIP_BUCKET - 1) / SIP_BUCKET;
    double part[SIP_THREADS], chunk_mass[SIP_THREADS], chunk_base[SIP_THREADS];
    for (int i = 0; i < pop; ++i) values[i] = fmaxf(input[i], 1e-30f);
    int certainty = 0;
    double scale;
    for (;;) { /* sip.cu:62-96 */
        double maxima[SIP_THREADS];
        for (int t = 0; t < SIP_THREADS; ++t) {
            double s = 0.0, m = 0.0;
            for (int i = t; i < pop; i += SIP_THREADS)
                if (values[i] > 0.f) {
                    const double v = fmax((double)values[i], 1e-30);
                    s = s + v;
                    m = fmax(m, v);
                }
            part[t] = s;
            maxima[t] = m;
        }
        const double total = block_sum(part);
        double maximum = 0.0;
        for (int t = 0; t < SIP_THREADS; ++t) maximum = fmax(maximum, maxima[t]);
        scale = (double)(samples - certainty) / total;
        int added = 0;
        if (maximum * scale >= 1.0) {
            for (int i = 0; i < pop; ++i)
                if (values[i] > 0.f && fmax((double)values[i], 1e-30) * scale >= 1.0) {
                    values[i] = -values[i];
                    ++added;
                }
        }
        certainty += added;
        if (added == 0) break;
    }
    const int chunk = ((buckets + SIP_THREADS - 1) / SIP_THREADS) * SIP_BUCKET; /* :99-101 */
    int last = pop - 1;
    while (last >= 0 && values[last] <= 0.f) --last;
    if (certainty != 0) { /* :108-124: certain ids first, ascending, weight 0 */
        int slot = 0;
        for (int i = 0; i < pop; ++i)
            if (values[i] < 0.f) {
                out[slot] = i;
                logs[slot++] = 0.f;
            }
    }
    for (int t = 0; t < SIP_THREADS; ++t) { /* :126-128 */
        const int begin = t * chunk;
        const int end = begin + chunk < pop ? begin + chunk : pop;
        double m = 0.0;
        for (int i = begin; i < end; ++i) m = m + (values[i] > 0.f ? (double)values[i] * scale : 0.0);
        chunk_mass[t] = m;
    }
    block_exclusive_sum(chunk_mass, chunk_base); /* :129-130 */
    const int residuals = (int)samples - certainty;
    prefix[buckets] = residuals;
    for (int t = 0; t < SIP_THREADS; ++t) { /* :137-141 */
        const int begin = t * chunk;
        const int end = begin + chunk < pop ? begin + chunk : pop;
        double cumulative = chunk_base[t];
        for (int i = begin; i < end; ++i) {
            if (i % SIP_BUCKET == 0) prefix[i / SIP_BUCKET] = i > last ? (double)residuals : cumulative;
            cumulative = cumulative + (values[i] > 0.f ? (double)values[i] * scale : 0.0);
        }
    }
    const double offset = (double)offset_f;
    for (int slot = 0; slot < residuals; ++slot) { /* :144-166 */
        const double threshold = offset + slot;
        int lower = 0, upper = buckets;
        while (lower < upper) {
            const int middle = (lower + upper + 1) / 2;
            if (prefix[middle] <= threshold)
                lower = middle;
            else
                upper = middle - 1;
        }
        const int bucket = lower < buckets - 1 ? lower : buckets - 1;
        double mass = prefix[bucket];
        int selected = last;
        const int stop = (bucket + 1) * SIP_BUCKET < pop ? (bucket + 1) * SIP_BUCKET : pop;
        for (int i = bucket * SIP_BUCKET; i < stop; ++i) {
            if (values[i] <= 0.f) continue;
            selected = i;
            mass = fma((double)values[i], scale, mass);
            if (mass > threshold) break;
        }
        out[certainty + slot] = selected;
        logs[certainty + slot] = (float)(-log2(fmax((double)input[selected], 1e-30) * scale));
    }
}

/*
 * scores [rows, pop] f32, offsets [rows] f32 -> ids [rows, samples] int32 and
 * log2(1/pi) weights [rows, samples] f32. Returns 0, or 1 on bad sizes.
 */
int orc_sip(const float *scores, const float *offsets, int64_t rows, int64_t population,
            int64_t samples, int32_t *ids, float *weights) {
    if (population <= 0 || samples <= 0 || samples >= population) return 1;
    const int pop = (int)population;
    const int buckets = (pop + SIP_BUCKET - 1) / SIP_BUCKET;
    int failed = 0;
#pragma omp parallel
    {
        float *values = malloc(sizeof(float) * (size_t)pop);
        double *prefix = malloc(sizeof(double) * (size_t)(buckets + 1));
#pragma omp for schedule(dynamic, 4)
        for (int64_t row = 0; row < rows; ++row) {
            if (!values || !prefix) {
#pragma omp atomic write
                failed = 1;
                continue;
            }
            sip_row(scores + row * pop, offsets[row], pop, samples, ids + row * samples, weights + row * samples,
                    values, prefix);
        }
        free(values);
        free(prefix);
    }
    return failed;
}

/* ---- weighted paged prefill (flashinfer_backend.py:30-59, :164-242) ---- */

/*
 * Exact (double) evaluation of the ABSipAttention variant:
 *   o_i = sum_j 2^{w_j} sum_{t in block j} e^{q_i.k_t/sqrt(128)} v_t / (same without v_t)
 *   lse_i = log2(sum_j 2^{w_j} sum_t e^{q_i.k_t/sqrt(128)})           (base 2)
 * q: float [bh, n, 128], k, v: float [bh, n_kv, 128] (bf16 inputs widened by
 * the caller); a -inf weight removes its block;
 * ids, logw: [rows, samples] per-head KV4 ids and log2 weights, rows = bh*qb.
 * out: float [bh, n, 128]; lse: float [bh, n] or NULL. Padded queries of the
 * last block are not produced (the reference computes and drops them).
 * row_list (optional, row_count entries) restricts the work to those rows;
 * outputs of other rows are left untouched.
 */
int orc_prefill_kv(const float *q, const float *k, const float *v, int64_t bh_count, int64_t n,
                   int64_t n_kv, const int32_t *ids, const float *logw, int64_t samples,
                   const int64_t *row_list, int64_t row_count, float *out, float *lse) {
    const int64_t qb = (n + QUERY_BLOCK - 1) / QUERY_BLOCK, fb = n_kv / KV_BLOCK;
    const int64_t keys = samples * KV_BLOCK;
    const double scale = 1.0 / sqrt((double)HEAD_DIM);
    const double ln2 = log(2.0);
    const int64_t total_rows = bh_count * qb;
    const int64_t count = row_list ? row_count : total_rows;
    for (int64_t r = 0; r < count; ++r) {
        const int64_t row = row_list ? row_list[r] : r;
        if (row < 0 || row >= total_rows) return 3;
        for (int64_t s = 0; s < samples; ++s)
            if (ids[row * samples + s] < 0 || ids[row * samples + s] >= fb) return 2;
    }
    int failed = 0;
#pragma omp parallel
    {
        double *logit = malloc(sizeof(double) * (size_t)keys);
        /* one task per (row, query): rows of a short list still spread over the threads */
#pragma omp for schedule(dynamic, 4)
        for (int64_t task = 0; task < count * QUERY_BLOCK; ++task) {
            const int64_t row = row_list ? row_list[task / QUERY_BLOCK] : task / QUERY_BLOCK;
            const int64_t bh = row / qb, blk = row % qb;
            const int64_t i = blk * QUERY_BLOCK + task % QUERY_BLOCK;
            if (i >= n) continue;
            if (!logit) {
#pragma omp atomic write
                failed = 1;
                continue;
            }
            const int32_t *rid = ids + row * samples;
            const float *rw = logw + row * samples;
            const float *qi = q + (bh * n + i) * HEAD_DIM;
            double mx = -INFINITY;
            for (int64_t s = 0; s < samples; ++s) {
                const int64_t j = rid[s];
                for (int t = 0; t < KV_BLOCK; ++t) {
                    const float *kt = k + (bh * n_kv + KV_BLOCK * j + t) * HEAD_DIM;
                    double dot = 0.0;
                    for (int d = 0; d < HEAD_DIM; ++d) dot += (double)qi[d] * (double)kt[d];
                    const double z = dot * scale + (double)rw[s] * ln2;
                    logit[s * KV_BLOCK + t] = z;
                    if (z > mx) mx = z;
                }
            }
            float *oi = out + (bh * n + i) * HEAD_DIM;
            if (mx == -INFINITY) {
                /* No listed key has a finite logit (every weight is -inf): the
                 * softmax is empty, so o = 0 and lse = -inf rather than the 0/0
                 * of the formula below. This convention is unpinned against the
                 * reference (no fixture covers it). */
                for (int d = 0; d < HEAD_DIM; ++d) oi[d] = 0.0f;
                if (lse) lse[bh * n + i] = -INFINITY;
                continue;
            }
            double acc[HEAD_DIM] = {0}, den = 0.0;
            for (int64_t s = 0; s < samples; ++s) {
                const int64_t j = rid[s];
                for (int t = 0; t < KV_BLOCK; ++t) {
                    const double p = exp(logit[s * KV_BLOCK + t] - mx);
                    const float *vt = v + (bh * n_kv + KV_BLOCK * j + t) * HEAD_DIM;
                    den += p;
                    for (int d = 0; d < HEAD_DIM; ++d) acc[d] += p * (double)vt[d];
                }
            }
            for (int d = 0; d < HEAD_DIM; ++d) oi[d] = (float)(acc[d] / den);
            if (lse) lse[bh * n + i] = (float)((mx + log(den)) / ln2);
        }
        free(logit);
    }
    return failed;
}

/* Q and K/V of the same length (the plan's case). */
int orc_prefill(const float *q, const float *k, const float *v, int64_t bh_count, int64_t n,
                const int32_t *ids, const float *logw, int64_t samples, const int64_t *row_list,
                int64_t row_count, float *out, float *lse) {
    return orc_prefill_kv(q, k, v, bh_count, n, n, ids, logw, samples, row_list, row_count, out, lse);
}
