/*
 * Oracle: tail-biting tile Viterbi in FP32 C -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the reference's tile quantizer pass structure
 * (qsrt/csrc/qsrt_quantize_tiles_kernel.cuh:79-499 and
 * qsrt/csrc/qsrt_quantize_tiles_k2_kernel.cuh:233-365), parametric in the
 * codeword width L (16 in production), the branch bits K, the tile length
 * T (256) and the tail-bite context C, so that tiny trellises can be
 * checked by exhaustive search.
 *
 * Arithmetic contract (this is what the HIP kernel must reproduce bit for
 * bit; the reference kernels use FP16 and differ by design):
 *   d = label - x                        (FP32 subtract)
 *   c = fmaf(d, d, predecessor_cost)     (one rounding; step 0 adds +0)
 *   per-state choice: lowest predecessor index k among equal minima
 *   boundary choice:  lowest state index among equal minima
 *   unreachable edges carry +inf (constrained first step only).
 * Built with -ffp-contract=off and without fast-math.  Steps after the first
 * run on AVX2 (sixteen states at a time, the same operations per lane); the
 * scalar loop below is the definition and a test compares the two bit for
 * bit.
 *
 * Trellis: codeword w has L bits; state = w & (2^(L-K) - 1); the codeword
 * entering state s from predecessor choice k is (k << (L-K)) | s and that
 * predecessor state is (k << (L-2K)) | (s >> K).
 *
 * Passes per tile (reference qsrt_quantize_tiles_kernel.cuh:494-499):
 *   1. primer: positions T-C .. T-1, 0 .. C-1 from a free start, decisions
 *      kept for positions 0 .. C-1;
 *   2. boundary = argmin of the primer's final costs (boundary_lag = 0, the
 *      K2 kernel, qsrt_quantize_tiles_k2_kernel.cuh:274-325) or of the
 *      costs one step earlier (boundary_lag = 1, what the generic kernel
 *      reads after its last buffer swap, qsrt_quantize_tiles_kernel.cuh:360-441);
 *   3. trace back to the state before position 0 (end_state);
 *   4. constrained pass over positions 0 .. T-1 whose first step only admits
 *      predecessor end_state;
 *   5. trace back from end_state at position T-1, emitting codewords and
 *      labels (qsrt_quantize_tiles_kernel.cuh:443-487).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef __AVX2__
#include <immintrin.h>
#endif

#ifdef _OPENMP
#include <omp.h>
#endif

typedef struct {
    int L, K, T, S, P;
    float *a, *b;      /* cost ping-pong, S floats each */
    uint8_t *dec;      /* T * S decisions */
} vt_ctx;

/* The vector path (AVX2 + FMA, sixteen consecutive states at a time) computes
 * exactly the scalar path's values: the same subtract, one fused multiply-add
 * per edge, and a strict less-than that keeps the lowest predecessor index on
 * ties (and, like the scalar compare, never replaces a value by a NaN).
 * qsrt_oracle_set_vector(0) selects the scalar path (tests compare the two). */
static int vt_use_vector = 1;

void qsrt_oracle_set_vector(int enable) { vt_use_vector = enable != 0; }

/* The OpenMP team size a call with n_threads = 0 uses (1 without OpenMP). */
int qsrt_oracle_default_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

#ifdef __AVX2__
/* predecessor costs of states s0 .. s0+7 (s0 a multiple of 8) for choice k */
static inline __m256 vt_pred8(const float *prev, int k, int q0, int K, int pred_shift)
{
    const float *pp = prev + (k << pred_shift) + q0;
    if (K >= 3) return _mm256_set1_ps(pp[0]);
    if (K == 2) return _mm256_set_m128(_mm_set1_ps(pp[1]), _mm_set1_ps(pp[0]));
    return _mm256_setr_ps(pp[0], pp[0], pp[1], pp[1], pp[2], pp[2], pp[3], pp[3]);
}

static inline void vt_store_dec8(uint8_t *drow, int s0, __m256i arg)
{
    /* eight decisions (< 64) narrowed to bytes */
    const __m128i h = _mm_packs_epi32(_mm256_castsi256_si128(arg), _mm256_extracti128_si256(arg, 1));
    _mm_storel_epi64((__m128i *)(drow + s0), _mm_packus_epi16(h, h));
}

/* costs of the 16 states s0 .. s0+15 (s0 a multiple of 16) at a step after the
 * first: two independent groups of eight, so the compare/blend chains of the
 * two overlap */
static void vt_step16(const float *lab, const float *prev, float *next, uint8_t *drow, int record, float w, int s0,
                      int K, int P, int word_shift, int pred_shift)
{
    const __m256 wv = _mm256_set1_ps(w);
    const int qa = s0 >> K, qb = (s0 + 8) >> K;
    __m256 best_a = _mm256_setzero_ps(), best_b = _mm256_setzero_ps();
    __m256i arg_a = _mm256_setzero_si256(), arg_b = _mm256_setzero_si256();
    for (int k = 0; k < P; ++k) {
        const float *lk = lab + ((size_t)k << word_shift) + s0;
        const __m256 da = _mm256_sub_ps(_mm256_loadu_ps(lk), wv);
        const __m256 db = _mm256_sub_ps(_mm256_loadu_ps(lk + 8), wv);
        const __m256 ca = _mm256_fmadd_ps(da, da, vt_pred8(prev, k, qa, K, pred_shift));
        const __m256 cb = _mm256_fmadd_ps(db, db, vt_pred8(prev, k, qb, K, pred_shift));
        if (k == 0) {
            best_a = ca;
            best_b = cb;
        } else {
            const __m256 kv = _mm256_castsi256_ps(_mm256_set1_epi32(k));
            const __m256 lta = _mm256_cmp_ps(ca, best_a, _CMP_LT_OQ);
            const __m256 ltb = _mm256_cmp_ps(cb, best_b, _CMP_LT_OQ);
            best_a = _mm256_blendv_ps(best_a, ca, lta);
            best_b = _mm256_blendv_ps(best_b, cb, ltb);
            arg_a = _mm256_castps_si256(_mm256_blendv_ps(_mm256_castsi256_ps(arg_a), kv, lta));
            arg_b = _mm256_castps_si256(_mm256_blendv_ps(_mm256_castsi256_ps(arg_b), kv, ltb));
        }
    }
    _mm256_storeu_ps(next + s0, best_a);
    _mm256_storeu_ps(next + s0 + 8, best_b);
    if (record) {
        vt_store_dec8(drow, s0, arg_a);
        vt_store_dec8(drow, s0 + 8, arg_b);
    }
}
#endif

/* One forward pass; returns the buffer holding the final costs and, via
 * *penult, the buffer holding the costs one step earlier.  pre_state < 0
 * starts free (every state at cost 0); otherwise the first step admits only
 * predecessor pre_state, carrying cost pre_cost. */
static float *vt_forward(vt_ctx *c, const float *lab, const float *x, int roll, int steps,
                         int pre_state, float pre_cost, int trace_start, float **penult)
{
    const int S = c->S, P = c->P, K = c->K, L = c->L;
    const int pred_shift = L - 2 * K, word_shift = L - K;
    float *prev = c->a, *next = c->b;
    for (int i = 0; i < steps; ++i) {
        const int pos = (i + roll) % c->T;
        const float w = x[pos];
        const int record = i >= trace_start;
        uint8_t *drow = c->dec + (size_t)pos * S;
#ifdef __AVX2__
        if (i > 0 && vt_use_vector && S % 16 == 0) {
            for (int s0 = 0; s0 < S; s0 += 16)
                vt_step16(lab, prev, next, drow, record, w, s0, K, P, word_shift, pred_shift);
            float *t = prev;
            prev = next;
            next = t;
            continue;
        }
#endif
        for (int s = 0; s < S; ++s) {
            const int q = s >> K;
            float best = 0.0f;
            int arg = 0;
            for (int k = 0; k < P; ++k) {
                const float d = lab[(k << word_shift) | s] - w;
                float cost;
                if (i == 0) {
                    const int pred = (k << pred_shift) | q;
                    cost = pre_state < 0 ? fmaf(d, d, 0.0f) : pred == pre_state ? fmaf(d, d, pre_cost) : INFINITY;
                } else {
                    cost = fmaf(d, d, prev[(k << pred_shift) | q]);
                }
                if (k == 0 || cost < best) {
                    best = cost;
                    arg = k;
                }
            }
            next[s] = best;
            if (record) drow[s] = (uint8_t)arg;
        }
        float *t = prev;
        prev = next;
        next = t;
    }
    *penult = next;
    return prev;
}

static int vt_argmin(const float *cost, int S)
{
    int arg = 0;
    for (int s = 1; s < S; ++s)
        if (cost[s] < cost[arg]) arg = s;
    return arg;
}

static int vt_trace(const vt_ctx *c, int roll, int steps, int edge, const float *lab,
                    uint16_t *states, float *recon)
{
    const int K = c->K, pred_shift = c->L - 2 * c->K;
    for (int i = steps - 1; i >= 0; --i) {
        const int pos = (i + roll) % c->T;
        const int k = c->dec[(size_t)pos * c->S + edge];
        const int prev = (k << pred_shift) | (edge >> K);
        if (states) {
            const int word = (prev << K) | edge;
            states[pos] = (uint16_t)word;
            recon[pos] = lab[word];
        } else if (pos == 0) {
            return prev;
        }
        edge = prev;
    }
    return edge;
}

static int vt_ctx_init(vt_ctx *c, int L, int K, int T)
{
    c->L = L; c->K = K; c->T = T; c->S = 1 << (L - K); c->P = 1 << K;
    c->a = (float *)malloc(sizeof(float) * c->S);
    c->b = (float *)malloc(sizeof(float) * c->S);
    c->dec = (uint8_t *)calloc((size_t)T * c->S, 1);
    return c->a && c->b && c->dec;
}

static void vt_ctx_free(vt_ctx *c)
{
    free(c->a);
    free(c->b);
    free(c->dec);
}

/*
 * tiles, recon: [n_tiles, T] float; states: [n_tiles, T] uint16;
 * labels: [2^L] float, state(codeword)-indexed; boundary (optional):
 * [n_tiles] int32 receiving end_state.  Returns 0, or -1 on bad arguments,
 * -2 on allocation failure.
 */
int qsrt_oracle_viterbi(const float *tiles, float *recon, uint16_t *states, int64_t n_tiles,
                        int L, int K, int T, int C, const float *labels, int boundary_lag,
                        int32_t *boundary, int n_threads)
{
    if (L < 2 || L > 16 || K < 1 || 2 * K > L || T < 2 || C < 1 || 2 * C > T ||
        (boundary_lag != 0 && boundary_lag != 1) || n_tiles < 0)
        return -1;
    int failed = 0;
    /* the thread count applies to this call's parallel region only (omp_set_num_threads would change the
     * process-wide default for every later call that passes 0) */
#ifdef _OPENMP
    const int team = n_threads > 0 ? n_threads : omp_get_max_threads();
#else
    const int team = 1;
    (void)n_threads;
#endif
#pragma omp parallel num_threads(team) reduction(| : failed)
    {
        vt_ctx c;
        if (!vt_ctx_init(&c, L, K, T)) failed = 1;
#pragma omp for schedule(dynamic, 1)
        for (int64_t t = 0; t < n_tiles; ++t) {
            if (failed) continue;
            const float *x = tiles + t * T;
            float *penult;
            float *fin = vt_forward(&c, labels, x, T - C, 2 * C, -1, 0.0f, C, &penult);
            const int start = vt_argmin(boundary_lag ? penult : fin, c.S);
            const int end_state = vt_trace(&c, T - C, 2 * C, start, labels, NULL, NULL);
            vt_forward(&c, labels, x, 0, T, end_state, 0.0f, 0, &penult);
            vt_trace(&c, 0, T, end_state, labels, states + t * T, recon + t * T);
            if (boundary) boundary[t] = end_state;
        }
        vt_ctx_free(&c);
    }
    return failed ? -2 : 0;
}

/*
 * The boundary choice of one tile (steps 1-3 above) laid open: cost [S]
 * receives the primer costs that the boundary argmin reads (the final ones,
 * or those one step earlier when boundary_lag = 1), final [S] (optional) the
 * final primer costs, and end_of [S] the end_state that each state's primer
 * survivor traces back to.  Returns 0, -1 on bad arguments, -2 on allocation
 * failure.
 */
int qsrt_oracle_viterbi_boundary(const float *tile, int L, int K, int T, int C, const float *labels,
                                 int boundary_lag, float *cost, float *final, int32_t *end_of)
{
    if (L < 2 || L > 16 || K < 1 || 2 * K > L || T < 2 || C < 1 || 2 * C > T ||
        (boundary_lag != 0 && boundary_lag != 1))
        return -1;
    vt_ctx c;
    int rc = 0;
    if (vt_ctx_init(&c, L, K, T)) {
        float *penult;
        const float *fin = vt_forward(&c, labels, tile, T - C, 2 * C, -1, 0.0f, C, &penult);
        memcpy(cost, boundary_lag ? penult : fin, sizeof(float) * c.S);
        if (final) memcpy(final, fin, sizeof(float) * c.S);
        for (int s = 0; s < c.S; ++s)
            end_of[s] = vt_trace(&c, T - C, 2 * C, s, labels, NULL, NULL);
    } else {
        rc = -2;
    }
    vt_ctx_free(&c);
    return rc;
}

/*
 * The primer restricted to paths whose state before position 0 is e:
 * through [S] receives, per final state, the cost of the best primer path
 * through e, computed with the primer's own operations in the primer's
 * order, so through[s] == final[s] exactly when state s's primer survivor
 * passes through e (ties included) and through[s] > final[s] otherwise.
 * Two encodes of nearly equal targets pick different end_states when, for
 * the state the boundary argmin picks, a path through another boundary
 * state costs nearly the same; this measures that margin.  Returns 0, -1 on
 * bad arguments, -2 on allocation failure.
 */
int qsrt_oracle_viterbi_primer_through(const float *tile, int L, int K, int T, int C, const float *labels,
                                       int e, float *through)
{
    if (L < 2 || L > 16 || K < 1 || 2 * K > L || T < 2 || C < 1 || 2 * C > T || e < 0 || e >= (1 << (L - K)))
        return -1;
    vt_ctx c;
    int rc = 0;
    if (vt_ctx_init(&c, L, K, T)) {
        float *penult;
        const float *head = vt_forward(&c, labels, tile, T - C, C, -1, 0.0f, C, &penult);
        const float at_e = head[e];
        const float *fin = vt_forward(&c, labels, tile, 0, C, e, at_e, C, &penult);
        memcpy(through, fin, sizeof(float) * c.S);
    } else {
        rc = -2;
    }
    vt_ctx_free(&c);
    return rc;
}

/*
 * Steps 4-5 alone: the constrained pass and trace of each tile from a given
 * end_state (end_states [n_tiles], each < 2^(L-K)), i.e. the best tail-biting
 * path through that boundary state.  Returns 0, -1 on bad arguments, -2 on
 * allocation failure.
 */
int qsrt_oracle_viterbi_from(const float *tiles, float *recon, uint16_t *states, int64_t n_tiles,
                             int L, int K, int T, const float *labels, const int32_t *end_states,
                             int n_threads)
{
    if (L < 2 || L > 16 || K < 1 || 2 * K > L || T < 2 || n_tiles < 0)
        return -1;
    for (int64_t t = 0; t < n_tiles; ++t)
        if (end_states[t] < 0 || end_states[t] >= (1 << (L - K))) return -1;
    int failed = 0;
    /* the thread count applies to this call's parallel region only (omp_set_num_threads would change the
     * process-wide default for every later call that passes 0) */
#ifdef _OPENMP
    const int team = n_threads > 0 ? n_threads : omp_get_max_threads();
#else
    const int team = 1;
    (void)n_threads;
#endif
#pragma omp parallel num_threads(team) reduction(| : failed)
    {
        vt_ctx c;
        if (!vt_ctx_init(&c, L, K, T)) failed = 1;
#pragma omp for schedule(dynamic, 1)
        for (int64_t t = 0; t < n_tiles; ++t) {
            if (failed) continue;
            float *penult;
            vt_forward(&c, labels, tiles + t * T, 0, T, end_states[t], 0.0f, 0, &penult);
            vt_trace(&c, 0, T, end_states[t], labels, states + t * T, recon + t * T);
        }
        vt_ctx_free(&c);
    }
    return failed ? -2 : 0;
}
