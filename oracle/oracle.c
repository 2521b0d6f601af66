/*
 * CPU oracle for the denoiser attention block: packed signed-Q4 projection GEMMs and exact
 * (flash-equivalent) attention.  TEST INFRASTRUCTURE ONLY.
 *
 * This file restates the reference algorithms in plain C so that the HIP kernels can be checked
 * against them.  It is imported only by tests/, by __graft_entry__.smoke() and by bench.py's
 * cpu_baseline leg; the product library (burn_image_amd/libbiq.so) never links or calls it.
 *
 * Every function cites the reference file:line it follows (paths relative to the reference repo
 * root).  Functions marked "CPU BASELINE" restate Burn's NdArray CPU path (dequantize, then f32
 * matmul; query-chunked f32 softmax attention) and are the CPU leg timed by bench.py.
 *
 * Parity pins (see tests/test_oracle_*.py): the Q4S quantizers are checked against the reference's
 * known-answer probe (exactly quantizable weights), its round-trip gates and its importer size /
 * dtype contracts; the GEMM against an independent numpy float64 product and the exact KAT;
 * attention against closed forms (S_kv = 1, constant keys, constant values), a numpy dense
 * softmax, chunked == dense, GQA == materialised expansion, causal-prefix and segment
 * non-interaction invariants; RoPE against math.cos/sin at known phases; RMSNorm against a
 * numpy restatement and the scale-invariance identity.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_OK 0
#define ORC_ERR 1

/* ------------------------------------------------------------------------------------------ */
/* Q4S formats                                                                                */
/* ------------------------------------------------------------------------------------------ */

/* Sign-extend one stored nibble: (v ^ 8) - 8.  The stored nibble is `(q as u8) & 0x0f`
 * (crates/burn_boogu/src/artifacts.rs:7273,7370), i.e. two's complement, so 0x8 decodes to -8. */
static inline int sext4(uint32_t v) { return (int)((v ^ 8u) & 15u) - 8; }

/* Rust `f32::round`: half away from zero.  `(x * inverse).round().clamp(-7, 7) as i8`
 * (artifacts.rs:7272,7354). */
static inline int quantize_one(float value, float inverse) {
    float r = roundf(value * inverse);
    if (r < -7.0f) r = -7.0f;
    if (r > 7.0f) r = 7.0f;
    return (int)r;
}

/* Scale rule shared by both quantizers: alpha = max|w| folded from 0.0 with f32::max;
 * scale = f32::MIN_POSITIVE if alpha == 0 else alpha / 7 (artifacts.rs:7262-7270,7345-7353). */
static inline float q4_scale(float alpha) { return alpha == 0.0f ? FLT_MIN : alpha / 7.0f; }

/* Block choice of the Boogu row layout: the largest of 128, 64, 32, 16, 8 dividing K, and N must
 * be a multiple of 8 (artifacts.rs:519-523, 7320-7336).  Returns 0 if none applies. */
int orc_q4_kn_block(int64_t K, int64_t N) {
    static const int groups[5] = {128, 64, 32, 16, 8};
    if (K <= 0 || N <= 0 || N % 8 != 0) return 0;
    for (int i = 0; i < 5; ++i)
        if (K % groups[i] == 0) return groups[i];
    return 0;
}

/* quantize_row_layout_q4s_block_up_to128_f32 (artifacts.rs:7296-7388).
 * w: logical [K, N] row-major f32 ([input, output]).  words: [K/8, N] u32, word (kw, n) holds
 * k = 8*kw + lane at bits 4*lane..4*lane+3.  scales: [K/blk, N] f32.  Returns ORC_ERR for
 * shapes without an exact block or for non-finite input, exactly where the reference errors. */
int orc_q4_quantize_kn(const float *w, int64_t K, int64_t N, uint32_t *words, float *scales,
                       int *block_out) {
    int blk = orc_q4_kn_block(K, N);
    if (blk == 0) return ORC_ERR;
    for (int64_t i = 0; i < K * N; ++i)
        if (!isfinite(w[i])) return ORC_ERR;
    int8_t *q = (int8_t *)malloc((size_t)(K * N));
    if (!q) return ORC_ERR;
    for (int64_t b = 0; b < K / blk; ++b) {
        for (int64_t n = 0; n < N; ++n) {
            float alpha = 0.0f;
            for (int64_t k = b * blk; k < (b + 1) * blk; ++k) {
                float a = fabsf(w[k * N + n]);
                alpha = alpha > a ? alpha : a;
            }
            float scale = q4_scale(alpha);
            scales[b * N + n] = scale;
            float inverse = 1.0f / scale;
            for (int64_t k = b * blk; k < (b + 1) * blk; ++k)
                q[k * N + n] = (int8_t)quantize_one(w[k * N + n], inverse);
        }
    }
    for (int64_t kw = 0; kw < K / 8; ++kw)
        for (int64_t n = 0; n < N; ++n) {
            uint32_t word = 0;
            for (int lane = 0; lane < 8; ++lane)
                word |= ((uint32_t)(uint8_t)q[(8 * kw + lane) * N + n] & 0x0fu) << (4 * lane);
            words[kw * N + n] = word;
        }
    free(q);
    if (block_out) *block_out = blk;
    return ORC_OK;
}

/* quantize_q4s_block128_f32 (artifacts.rs:7203-7288): contiguous 128-value chunks of the
 * flattened tensor, eight values per little-endian word along the last axis.  values: [rows,
 * inner] with inner % 128 == 0 (for Qwen weights rows = N, inner = K).  words: [rows, inner/8];
 * scales: [rows, inner/128] (chunk order). */
int orc_q4_quantize_nk(const float *values, int64_t rows, int64_t inner, uint32_t *words,
                       float *scales) {
    if (rows <= 0 || inner <= 0 || inner % 128 != 0) return ORC_ERR;
    int64_t total = rows * inner;
    for (int64_t c = 0; c < total / 128; ++c) {
        const float *blk = values + c * 128;
        for (int i = 0; i < 128; ++i)
            if (!isfinite(blk[i])) return ORC_ERR;
        float alpha = 0.0f;
        for (int i = 0; i < 128; ++i) {
            float a = fabsf(blk[i]);
            alpha = alpha > a ? alpha : a;
        }
        float scale = q4_scale(alpha);
        scales[c] = scale;
        float inverse = 1.0f / scale;
        for (int wv = 0; wv < 16; ++wv) {
            uint32_t word = 0;
            for (int lane = 0; lane < 8; ++lane) {
                int qv = quantize_one(blk[wv * 8 + lane], inverse);
                word |= ((uint32_t)(uint8_t)(int8_t)qv & 0x0fu) << (4 * lane);
            }
            words[c * 16 + wv] = word;
        }
    }
    return ORC_OK;
}

/* Decode one signed nibble of either layout.
 * layout 1 (Boogu, PackedU32(1), block [blk,1]): words [K/8, N], scales [K/blk, N].
 * layout 0 (Qwen, PackedU32(0), block [blk]):    words [N, K/8], scales [N, K/blk]. */
static inline int q4_at(const uint32_t *words, int layout, int64_t K, int64_t N, int64_t k,
                        int64_t n) {
    uint32_t word = layout == 1 ? words[(k / 8) * N + n] : words[n * (K / 8) + k / 8];
    return sext4(word >> (4 * (k % 8)));
}
static inline float scale_at(const float *scales, int layout, int block, int64_t K, int64_t N,
                             int64_t k, int64_t n) {
    return layout == 1 ? scales[(k / block) * N + n] : scales[n * (K / block) + k / block];
}

/* Dequantization: `f32::from(q) * scale`, one IEEE f32 multiply per element
 * (artifacts.rs:10434-10440).  Output is the tensor's logical shape: [K, N] for layout 1 and
 * [N, K] for layout 0. */
void orc_q4_dequant(const uint32_t *words, const float *scales, int layout, int block, int64_t K,
                    int64_t N, float *out) {
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) {
            float v = (float)q4_at(words, layout, K, N, k, n) * scale_at(scales, layout, block, K, N, k, n);
            if (layout == 1) out[k * N + n] = v;
            else out[n * K + k] = v;
        }
}

/* Y[rows, N] = X[rows, K] . W where W = dequant(words) in logical [K, N] orientation, for a subset
 * of rows (row_index[r]; NULL = rows 0..nrows-1), accumulated in double.  This is the float64
 * statement of `linear_forward` / `qwen_linear_forward` over a Q4S weight
 * (crates/burn_boogu/src/model/linear.rs:14-37; crates/burn_qwen3_vl/src/linear.rs:107-140),
 * where the Qwen [N, K] weight is consumed transposed.  bias may be NULL. */
void orc_q4_linear_f64(const float *x, int64_t K, const int64_t *row_index, int64_t nrows,
                       const uint32_t *words, const float *scales, int layout, int block,
                       int64_t N, const float *bias, double *y) {
    float *wdq = (float *)malloc(sizeof(float) * (size_t)(K * N));
    /* dequantized [K, N] */
    #pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n)
            wdq[k * N + n] = (float)q4_at(words, layout, K, N, k, n) * scale_at(scales, layout, block, K, N, k, n);
    #pragma omp parallel for schedule(dynamic, 1)
    for (int64_t r = 0; r < nrows; ++r) {
        int64_t m = row_index ? row_index[r] : r;
        double *acc = y + r * N;
        for (int64_t n = 0; n < N; ++n) acc[n] = bias ? (double)bias[n] : 0.0;
        const float *xr = x + m * K;
        for (int64_t k = 0; k < K; ++k) {
            double xv = xr[k];
            const float *wr = wdq + k * N;
            for (int64_t n = 0; n < N; ++n) acc[n] += xv * (double)wr[n];
        }
    }
    free(wdq);
}

/* CPU BASELINE (restated Burn NdArray `q_matmul`): dequantize the whole weight to f32, then an f32
 * matmul with f32 accumulation, rows in parallel.  Burn's CPU backend lowers q_matmul to the
 * default dequantize-then-matmul (patches/burn-cubecl-0.21.0/src/ops/qtensor.rs:352-356 routes
 * every non-packed case to the default; burn-ndarray 0.21.0 uses matrixmultiply's SGEMM).
 * Returns the number of threads used. */
int orc_cpu_q4_linear_f32(const float *x, int64_t M, int64_t K, const uint32_t *words,
                          const float *scales, int layout, int block, int64_t N, float *y) {
    float *wdq = (float *)malloc(sizeof(float) * (size_t)(K * N));
    #pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n)
            wdq[k * N + n] = (float)q4_at(words, layout, K, N, k, n) * scale_at(scales, layout, block, K, N, k, n);
    const int64_t MB = 32, KB = 256, NB = 512;
    #pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int64_t m0 = 0; m0 < M; m0 += MB)
        for (int64_t n0 = 0; n0 < N; n0 += NB) {
            int64_t m1 = m0 + MB < M ? m0 + MB : M, n1 = n0 + NB < N ? n0 + NB : N;
            for (int64_t m = m0; m < m1; ++m)
                for (int64_t n = n0; n < n1; ++n) y[m * N + n] = 0.0f;
            for (int64_t k0 = 0; k0 < K; k0 += KB) {
                int64_t k1 = k0 + KB < K ? k0 + KB : K;
                for (int64_t m = m0; m < m1; ++m) {
                    float *yr = y + m * N;
                    for (int64_t k = k0; k < k1; ++k) {
                        float xv = x[m * K + k];
                        const float *wr = wdq + k * N;
                        for (int64_t n = n0; n < n1; ++n) yr[n] += xv * wr[n];
                    }
                }
            }
        }
    free(wdq);
    int threads = 1;
#ifdef _OPENMP
    threads = omp_get_max_threads();
#endif
    return threads;
}

/* ------------------------------------------------------------------------------------------ */
/* Attention                                                                                  */
/* ------------------------------------------------------------------------------------------ */

/* effective_portable_query_chunk_size (crates/burn_boogu/src/model/attention.rs:36-45). */
int64_t orc_effective_query_chunk(int64_t query_len, int64_t requested) {
    const int64_t dflt = 128, parts = 4;
    if (requested <= 0 || query_len <= 0) return 0;
    if (query_len <= dflt) return requested < query_len ? requested : query_len;
    int64_t cap = (query_len + parts - 1) / parts;
    if (cap < dflt) cap = dflt;
    return requested < cap ? requested : cap;
}

/* Segment of position i: cu_seqlens[s] <= i < cu_seqlens[s+1]. */
static int64_t segment_of(const int32_t *cu, int64_t nseg, int64_t i) {
    int64_t lo = 0, hi = nseg - 1;
    while (lo < hi) {
        int64_t mid = (lo + hi + 1) / 2;
        if (cu[mid] <= i) lo = mid; else hi = mid - 1;
    }
    return lo;
}

/* Visibility of key j from query i.  Causal follows Qwen's per-chunk `triu_mask(start + 1)`
 * (key j masked iff j > i; crates/burn_qwen3_vl/src/text.rs:146-158); segments follow the
 * per-frame block-diagonal loop (crates/burn_qwen3_vl/src/vision.rs:344-386): key visible iff it
 * lies in the query's segment. */
static inline int visible(int64_t i, int64_t j, int causal, const int32_t *cu, int64_t nseg) {
    if (causal && j > i) return 0;
    if (cu && segment_of(cu, nseg, i) != segment_of(cu, nseg, j)) return 0;
    return 1;
}

/* Exact attention softmax(Q K^T * scale) V in double for selected query rows.
 * Layout: q [B, Hq, Sq, D], k [B, Hkv, Skv, D], v [B, Hkv, Skv, Dv] contiguous f32 (inputs already
 * rounded to the kernel's input dtype), out [B, Hq, nrows, Dv] double.  GQA maps query head h to
 * key/value head h / (Hq / Hkv) (attention.rs:67-105 materialised `repeat_dim`).  Masked scores are
 * excluded exactly (Qwen fills -1e30 before softmax, whose weight underflows to 0 in f32).
 * key_valid: NULL or [B, Skv] bytes, nonzero = the key may be attended: Qwen's key-padding
 * `attention_mask`, OR-ed into the causal mask as `valid.bool_not()` broadcast over queries
 * (crates/burn_qwen3_vl/src/text.rs:163-176).  A row left with no visible key gets, with
 * fill_mean, the mean of V over all Skv keys (softmax of a row filled with -1e30 everywhere is
 * uniform, text.rs:177-182), and zeros without it.
 * rows: query indices evaluated (NULL = all Sq). */
void orc_attention_f64(const float *q, const float *k, const float *v, int64_t B, int64_t Hq,
                       int64_t Hkv, int64_t Sq, int64_t Skv, int64_t D, int64_t Dv, double scale,
                       int causal, const int32_t *cu_seqlens, int64_t nseg,
                       const uint8_t *key_valid, int fill_mean, const int64_t *rows,
                       int64_t nrows, double *out) {
    int64_t group = Hq / Hkv;
    #pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int64_t bh = 0; bh < B * Hq; ++bh)
        for (int64_t r = 0; r < nrows; ++r) {
            int64_t b = bh / Hq, h = bh % Hq, hk = h / group;
            int64_t i = rows ? rows[r] : r;
            const float *qr = q + ((b * Hq + h) * Sq + i) * D;
            const float *kb = k + (b * Hkv + hk) * Skv * D;
            const float *vb = v + (b * Hkv + hk) * Skv * Dv;
            double *o = out + ((b * Hq + h) * nrows + r) * Dv;
            double *s = (double *)malloc(sizeof(double) * (size_t)Skv);
            double mx = -INFINITY;
            for (int64_t j = 0; j < Skv; ++j) {
                if (!visible(i, j, causal, cu_seqlens, nseg) ||
                    (key_valid && !key_valid[b * Skv + j])) { s[j] = -INFINITY; continue; }
                double acc = 0.0;
                for (int64_t d = 0; d < D; ++d) acc += (double)qr[d] * (double)kb[j * D + d];
                s[j] = acc * scale;
                if (s[j] > mx) mx = s[j];
            }
            double denom = 0.0;
            for (int64_t j = 0; j < Skv; ++j) {
                s[j] = s[j] == -INFINITY ? 0.0 : exp(s[j] - mx);
                denom += s[j];
            }
            for (int64_t d = 0; d < Dv; ++d) o[d] = 0.0;
            if (mx == -INFINITY) {  /* no visible key */
                if (fill_mean)
                    for (int64_t j = 0; j < Skv; ++j)
                        for (int64_t d = 0; d < Dv; ++d) o[d] += (double)vb[j * Dv + d] / (double)Skv;
                free(s);
                continue;
            }
            for (int64_t j = 0; j < Skv; ++j) {
                if (s[j] == 0.0) continue;
                double p = s[j] / denom;
                for (int64_t d = 0; d < Dv; ++d) o[d] += p * (double)vb[j * Dv + d];
            }
            free(s);
        }
}

/* CPU BASELINE (restated portable path): `query_chunked_attention` (attention.rs:875-914) over
 * chunks of `effective_portable_query_chunk_size`, each chunk the dense f32 attention of Burn's
 * `attention_fallback`: f32 scores Q K^T * scale, row softmax, P V.  Layout as
 * orc_attention_f64 with Hq == Hkv expected (GQA expansion is a view here), f32 out
 * [B, Hq, Sq, Dv].  q_rows limits the evaluated query range to [0, q_rows) (bench sampling).
 * Returns the number of threads used. */
int orc_cpu_attention_f32(const float *q, const float *k, const float *v, int64_t B, int64_t Hq,
                          int64_t Hkv, int64_t Sq, int64_t Skv, int64_t D, int64_t Dv,
                          float scale, int64_t requested_chunk, int64_t q_rows, float *out) {
    int64_t chunk = orc_effective_query_chunk(Sq, requested_chunk);
    int64_t group = Hq / Hkv;
    int64_t nchunks = (q_rows + chunk - 1) / chunk;
    #pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int64_t bh = 0; bh < B * Hq; ++bh)
        for (int64_t c = 0; c < nchunks; ++c) {
            int64_t b = bh / Hq, h = bh % Hq, hk = h / group;
            int64_t start = c * chunk, end = start + chunk < q_rows ? start + chunk : q_rows;
            const float *kb = k + (b * Hkv + hk) * Skv * D;
            const float *vb = v + (b * Hkv + hk) * Skv * Dv;
            float *srow = (float *)malloc(sizeof(float) * (size_t)Skv);
            for (int64_t i = start; i < end; ++i) {
                const float *qr = q + ((b * Hq + h) * Sq + i) * D;
                float mx = -INFINITY;
                for (int64_t j = 0; j < Skv; ++j) {
                    float acc = 0.0f;
                    const float *kr = kb + j * D;
                    for (int64_t d = 0; d < D; ++d) acc += qr[d] * kr[d];
                    srow[j] = acc * scale;
                    mx = srow[j] > mx ? srow[j] : mx;
                }
                float denom = 0.0f;
                for (int64_t j = 0; j < Skv; ++j) { srow[j] = expf(srow[j] - mx); denom += srow[j]; }
                float *o = out + ((b * Hq + h) * Sq + i) * Dv;
                for (int64_t d = 0; d < Dv; ++d) o[d] = 0.0f;
                for (int64_t j = 0; j < Skv; ++j) {
                    float p = srow[j] / denom;
                    const float *vr = vb + j * Dv;
                    for (int64_t d = 0; d < Dv; ++d) o[d] += p * vr[d];
                }
            }
            free(srow);
        }
    int threads = 1;
#ifdef _OPENMP
    threads = omp_get_max_threads();
#endif
    return threads;
}

/* ------------------------------------------------------------------------------------------ */
/* RoPE and RMSNorm                                                                           */
/* ------------------------------------------------------------------------------------------ */

/* rope_values (crates/burn_boogu/src/model/denoiser.rs:992-1034): per axis a, pair p, inverse
 * frequency theta^(-2p/dim_a) in f64; phase = id[a] * inv in f64; cos/sin in f64 then cast to f32,
 * each repeated for the two interleaved lanes of the pair.  ids: [S, 3] u32; cos/sin: [S, sum(dims)]. */
void orc_rope_values(const uint32_t *ids, int64_t S, const int64_t *axis_dims, double theta,
                     float *cos_out, float *sin_out) {
    int64_t head_dim = axis_dims[0] + axis_dims[1] + axis_dims[2];
    for (int64_t s = 0; s < S; ++s) {
        int64_t col = 0;
        for (int a = 0; a < 3; ++a) {
            int64_t dim = axis_dims[a];
            for (int64_t p = 0; p < dim / 2; ++p) {
                double inv = pow(theta, -((double)(2 * p)) / (double)dim);
                double phase = (double)ids[s * 3 + a] * inv;
                float c = (float)cos(phase), sn = (float)sin(phase);
                cos_out[s * head_dim + col] = c; cos_out[s * head_dim + col + 1] = c;
                sin_out[s * head_dim + col] = sn; sin_out[s * head_dim + col + 1] = sn;
                col += 2;
            }
        }
    }
}

/* Strict-F32 RMSNorm (crates/burn_boogu/src/model/norm.rs:28-35 via nn::RmsNorm; the fused
 * kernel statement crates/burn_boogu/src/model/native_flash.rs:424-441): rms = sqrt(sum(x^2)/D +
 * eps) in f32, y = x / rms * gamma.  x, y: [rows, D]. */
void orc_rms_norm_f32(const float *x, int64_t rows, int64_t D, const float *gamma, float eps,
                      float *y) {
    for (int64_t r = 0; r < rows; ++r) {
        double acc = 0.0;
        for (int64_t d = 0; d < D; ++d) acc += (double)x[r * D + d] * (double)x[r * D + d];
        float rms = sqrtf((float)acc / (float)D + eps);
        for (int64_t d = 0; d < D; ++d) y[r * D + d] = x[r * D + d] / rms * gamma[d];
    }
}

/* Boogu interleaved-pair RoPE (attention.rs:916-928): for pair (x0, x1) at lanes (2p, 2p+1),
 * y = x * cos + rotated * sin with rotated = (-x1, x0).  x, y: [rows, D]; cos/sin: [rows, D]. */
void orc_apply_rope_interleaved(const float *x, int64_t rows, int64_t D, const float *cs,
                                const float *sn, float *y) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t d = 0; d < D; ++d) {
            float rot = (d % 2 == 0) ? -x[r * D + d + 1] : x[r * D + d - 1];
            y[r * D + d] = x[r * D + d] * cs[r * D + d] + rot * sn[r * D + d];
        }
}

/* Qwen rotate_half RoPE (crates/burn_qwen3_vl/src/text.rs:407-440): rotated = cat(-x[h:], x[:h]),
 * y = x * cos + rotated * sin in f32. */
void orc_apply_rope_half(const float *x, int64_t rows, int64_t D, const float *cs,
                         const float *sn, float *y) {
    int64_t h = D / 2;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t d = 0; d < D; ++d) {
            float rot = d < h ? -x[r * D + d + h] : x[r * D + d - h];
            y[r * D + d] = x[r * D + d] * cs[r * D + d] + rot * sn[r * D + d];
        }
}
