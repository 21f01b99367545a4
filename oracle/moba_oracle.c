/*
 * Plain-C restatement of the MoBA pooling and gate -- TEST INFRASTRUCTURE.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker of the HIP kernels. It exists
 * because the torch oracle materialises a [S, num_blocks] score matrix,
 * which does not fit at S = 64K..512K; this one streams.
 *
 * Semantics restated:
 *   pool  : src/moba/naive.py:23-61 and src/moba/kernels/pooling.py:82-93 --
 *           block sum (exact, float64) -> float32 -> input dtype, then divide
 *           by the block's real occupancy in float32 and round to the dtype.
 *   gate  : src/moba/naive.py:64-146 -- candidates are blocks strictly before
 *           the query's own block, score = q . kbar (unscaled) rounded once
 *           to float32 and once to the dtype, the top past_blocks_selected()
 *           by (score desc, block id asc) are kept (the stable descending
 *           argsort of naive.py:124-127), the own block is added when forced,
 *           and ids are emitted ascending with -1 padding
 *           (src/moba/kernels/gating.py:300-335).
 *   varlen: src/moba/naive.py:149-189 -- every sequence gated alone with
 *           sequence-local block ids.
 *
 * Inputs are float32 arrays holding values already representable in the
 * input dtype (the caller widens bf16/fp16 losslessly). dtype codes:
 * 0 = bf16, 1 = fp16, 2 = fp32.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

static float round_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) {          /* inf / nan */
        if (u & 0x007fffffu) u |= 0x00400000u;
        u &= 0xffff0000u;
    } else {
        uint32_t lsb = (u >> 16) & 1u;
        u += 0x7fffu + lsb;
        u &= 0xffff0000u;
    }
    float r;
    memcpy(&r, &u, 4);
    return r;
}

/* Round-to-nearest-even to IEEE binary16, returned widened to float. */
static float round_fp16(float x) {
    if (isnan(x) || isinf(x)) return x;
    float ax = fabsf(x);
    if (ax >= 65520.0f) return copysignf(INFINITY, x);
    int e;
    frexpf(ax, &e);                       /* ax = m * 2^e, m in [0.5, 1) */
    int exp2u = e - 11;                   /* ulp exponent for 11-bit mantissa */
    if (exp2u < -24) exp2u = -24;         /* subnormal spacing 2^-24 */
    float scaled = ldexpf(ax, -exp2u);    /* exact: power-of-two scale */
    float r = nearbyintf(scaled);         /* default mode: ties to even */
    return copysignf(ldexpf(r, exp2u), x);
}

static float round_dtype(double x, int dtype) {
    float f = (float)x;
    if (dtype == 0) return round_bf16(f);
    if (dtype == 1) return round_fp16(f);
    return f;
}

/* k: [B, S, H, D] token-major; kbar: [B, H, nb, D] head-major. When
 * cu_seqlens is given, B = 1 on input and kbar is [n_seq, H, nb, D]. */
void oracle_pool(const float* k, int B, int S, int H, int D, int bs,
                 int dtype, const int32_t* cu, int n_seq, int nb,
                 float* kbar) {
    int rows = cu ? n_seq : B;
    for (int r = 0; r < rows; ++r) {
        int lo_seq = cu ? cu[r] : 0;
        int len = cu ? cu[r + 1] - cu[r] : S;
        int nblk = (len + bs - 1) / bs;
        for (int h = 0; h < H; ++h)
            for (int n = 0; n < nblk; ++n) {
                int lo = n * bs, hi = lo + bs < len ? lo + bs : len;
                for (int d = 0; d < D; ++d) {
                    double acc = 0.0;
                    for (int t = lo; t < hi; ++t) {
                        size_t tok = cu ? (size_t)(lo_seq + t)
                                        : (size_t)r * S + t;
                        acc += (double)k[(tok * H + h) * D + d];
                    }
                    float sum = round_dtype(acc, dtype);
                    float mean = sum / (float)(hi - lo);
                    kbar[(((size_t)r * H + h) * nb + n) * D + d] =
                        dtype == 2 ? mean : round_dtype(mean, dtype);
                }
            }
    }
}

/* Exact score, rounded once to float32 and once to the dtype. */
static float score(const float* q, const float* kb, int D, int dtype) {
    double acc = 0.0;
    for (int d = 0; d < D; ++d) acc += (double)q[d] * (double)kb[d];
    return round_dtype(acc, dtype);
}

/* Streaming top-`take` by (score desc, id asc). Blocks arrive in ascending
 * id order, so a later block must score strictly higher than the current
 * worst entry to enter, and among tied worst entries the highest id leaves.
 * This is exactly the prefix of a stable descending sort. */
static int topk_stream(const float* q, const float* kbase, int D, int ncand,
                       int take, int dtype, float* val, int* idx) {
    int cnt = 0;
    for (int j = 0; j < ncand; ++j) {
        float s = score(q, kbase + (size_t)j * D, D, dtype);
        if (isnan(s)) continue;
        if (cnt < take) {
            val[cnt] = s;
            idx[cnt] = j;
            ++cnt;
            continue;
        }
        int w = 0;
        for (int t = 1; t < cnt; ++t)
            if (val[t] < val[w] || (val[t] == val[w] && idx[t] > idx[w])) w = t;
        if (s > val[w]) {
            val[w] = s;
            idx[w] = j;
        }
    }
    return cnt;
}

static int cmp_int(const void* a, const void* b) {
    int x = *(const int*)a, y = *(const int*)b;
    return (x > y) - (x < y);
}

/* q: [B, S, Hq, D]; kbar: [rows, Hkv, nb, D]; out: [B, Hq, S, slots] int32.
 * take = past-block budget, cur = whether the own block is forced.
 * Queries with -inf scores (e.g. q containing -inf) are treated as absent
 * candidates, matching naive.py:142 (`selected &= is_past` drops -inf). */
void oracle_gate(const float* q, const float* kbar, int B, int S, int Hq,
                 int Hkv, int D, int nb, int bs, int take, int cur,
                 int slots, int dtype, const int32_t* cu, int n_seq,
                 int32_t* out) {
    int g = Hq / Hkv;
    int rows = cu ? n_seq : B;
#pragma omp parallel for schedule(dynamic, 64) collapse(2)
    for (int r = 0; r < rows; ++r) {
        for (int hq = 0; hq < Hq; ++hq) {
            int lo_seq = cu ? cu[r] : 0;
            int len = cu ? cu[r + 1] - cu[r] : S;
            int nblk_seq = (len + bs - 1) / bs;
            int budget = take < nblk_seq ? take : nblk_seq;
            float* val = (float*)malloc(sizeof(float) * (budget + 1));
            int* idx = (int*)malloc(sizeof(int) * (budget + 2 + slots));
            const float* kb = kbar + ((size_t)r * Hkv + hq / g) * nb * D;
            for (int t = 0; t < len; ++t) {
                size_t tok = cu ? (size_t)(lo_seq + t) : (size_t)r * S + t;
                const float* qq = q + (tok * Hq + hq) * D;
                int own = t / bs;
                int cnt = topk_stream(qq, kb, D, own, budget, dtype, val, idx);
                /* drop -inf leftovers: naive.py:142 */
                int m = 0;
                for (int i = 0; i < cnt; ++i)
                    if (val[i] > -INFINITY) idx[m++] = idx[i];
                if (cur) idx[m++] = own;
                qsort(idx, m, sizeof(int), cmp_int);
                int32_t* o = out + (((size_t)(cu ? 0 : r) * Hq + hq) *
                                    (cu ? (size_t)S : (size_t)S) + tok -
                                    (cu ? 0 : (size_t)r * S)) * slots;
                for (int i = 0; i < slots; ++i) o[i] = i < m ? idx[i] : -1;
            }
            free(val);
            free(idx);
        }
    }
}


/* The gate of oracle_gate on a subset of a padded batch: query heads
 * [hq_lo, hq_hi) and the rows t = off, off + stride, ... of every batch row.
 * Parallel over those query rows, so one head of a 512K-token sequence is
 * checked in seconds. out: [B, hq_hi - hq_lo, ceil((S - off) / stride),
 * slots] int32. Same semantics as oracle_gate (src/moba/naive.py:64-146). */
void oracle_gate_strided(const float* q, const float* kbar, int B, int S,
                         int Hq, int Hkv, int D, int nb, int bs, int take,
                         int cur, int slots, int dtype, int hq_lo, int hq_hi,
                         int off, int stride, int32_t* out) {
    int g = Hq / Hkv;
    int nh = hq_hi - hq_lo;
    long nt = off < S ? (S - off + stride - 1) / stride : 0;
    long total = (long)B * nh * nt;
    int nblk = (S + bs - 1) / bs;
    int budget = take < nblk ? take : nblk;
#pragma omp parallel
    {
        float* val = (float*)malloc(sizeof(float) * (budget + 1));
        int* idx = (int*)malloc(sizeof(int) * (budget + 2 + slots));
#pragma omp for schedule(dynamic, 256)
        for (long i = 0; i < total; ++i) {
            long ti = i % nt;
            int h = (int)((i / nt) % nh) + hq_lo;
            int r = (int)(i / nt / nh);
            int t = off + (int)ti * stride;
            const float* kb = kbar + ((size_t)r * Hkv + h / g) * nb * D;
            const float* qq = q + (((size_t)r * S + t) * Hq + h) * D;
            int own = t / bs;
            int cnt = topk_stream(qq, kb, D, own, budget, dtype, val, idx);
            int m = 0;
            for (int j = 0; j < cnt; ++j)
                if (val[j] > -INFINITY) idx[m++] = idx[j];
            if (cur) idx[m++] = own;
            qsort(idx, m, sizeof(int), cmp_int);
            int32_t* o = out + (size_t)i * slots;
            for (int j = 0; j < slots; ++j) o[j] = j < m ? idx[j] : -1;
        }
        free(val);
        free(idx);
    }
}

int oracle_version(void) { return 2; }
