/*
 * spike_oracle.c -- CPU restatement of the spiking decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load this library, and only as the checker or
 * the timed CPU baseline; the product (spikeinfer_amd) never calls it.
 *
 * Each function restates the reference algorithm it names:
 *   orc_pack_rows      spikeinfer/kernels/packing.py:16-23, 84-111
 *   orc_unpack_rows    spikeinfer/kernels/packing.py:136-152
 *   orc_lif            spikeinfer/kernels/lif_triton.py:13-28, 96-105, 126-138
 *   orc_decode_attn    spikeinfer/kernels/spike_attention.py:86-150 (indexing,
 *                      masking, scale) with the softmax of its oracle
 *                      spike_attention.py:247-282, evaluated in float64 with
 *                      the true running maximum
 *   orc_decode_scores  spike_attention.py:108-120 (block walk, popcount)
 *   orc_lif_pack_write composition lif -> pack -> index_copy_ of
 *                      spikeinfer/modeling_fast.py:132-134 and
 *                      spikeinfer/attention.py:138-139, 146-149
 *
 * Build: gcc -O2 -fopenmp -ffp-contract=off -fPIC -shared (oracle/build.py).
 * -ffp-contract=off is load-bearing for orc_lif: PyTorch eager rounds the
 * multiply and the add of `beta*u + x` separately.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int orc_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
  return omp_get_max_threads();
#else
  (void)n;
  return 1;
#endif
}

/* bits: uint8 [rows, C] (nonzero = spike) -> int32 [rows, W]. */
void orc_pack_rows(const uint8_t *bits, int64_t rows, int C, int32_t *out) {
  const int W = (C + 31) / 32;
  for (int64_t r = 0; r < rows; ++r) {
    for (int w = 0; w < W; ++w) {
      uint32_t word = 0;
      for (int i = 0; i < 32; ++i) {
        const int c = 32 * w + i;
        if (c < C && bits[r * C + c]) word |= (uint32_t)1 << i;
      }
      out[r * W + w] = (int32_t)word;
    }
  }
}

void orc_unpack_rows(const int32_t *words, int64_t rows, int C, uint8_t *bits) {
  const int W = (C + 31) / 32;
  for (int64_t r = 0; r < rows; ++r)
    for (int c = 0; c < C; ++c)
      bits[r * C + c] = (uint8_t)(((uint32_t)words[r * W + c / 32] >> (c % 32)) & 1u);
}

/*
 * x float [T, M, N]; beta, thr float [N]; mem0 float [M, N] or NULL;
 * spikes uint8 [T, M, N]; u_out float [M, N] or NULL.
 */
void orc_lif(const float *x, int T, int64_t M, int N, const float *beta, const float *thr,
             const float *mem0, uint8_t *spikes, float *u_out) {
  const int64_t MN = M * N;
#pragma omp parallel for schedule(static)
  for (int64_t e = 0; e < MN; ++e) {
    const int n = (int)(e % N);
    float b = beta[n];
    b = b < 0.f ? 0.f : (b > 1.f ? 1.f : b); /* Tensor.clamp(0, 1) */
    const float th = thr[n];
    float u = mem0 ? mem0[e] : 0.f;
    for (int t = 0; t < T; ++t) {
      const float r = (u - th > 0.f) ? 1.f : 0.f; /* reset from the previous membrane */
      const float bu = b * u;
      const float s1 = bu + x[t * MN + e];
      u = s1 - r * th;
      spikes[t * MN + e] = (u - th > 0.f) ? 1 : 0;
    }
    if (u_out) u_out[e] = u;
  }
}

static inline int64_t slot_of(const int32_t *tables, int64_t maxb, int n, int p, int bs) {
  const int32_t phys = tables[(int64_t)n * maxb + p / bs];
  return (int64_t)phys * bs + p % bs;
}

/*
 * q int32 [T, N, Hq, W]; k, v int32 [T, Hkv, S, W]; tables int32 [N, maxb];
 * lens int32 [N]; out double [T, N, Hq, hd].  scale = 1/sqrt(hd).
 * A sequence with len <= 0 gets zeros (the product's documented choice).
 */
void orc_decode_attn(const int32_t *q, const int32_t *k, const int32_t *v, const int32_t *tables,
                     const int32_t *lens, int T, int N, int Hq, int Hkv, int hd, int bs,
                     int64_t maxb, int64_t S, double *out) {
  const int W = (hd + 31) / 32;
  const int nrep = Hq / Hkv;
  const double scale = 1.0 / sqrt((double)hd);
#pragma omp parallel for collapse(3) schedule(dynamic)
  for (int t = 0; t < T; ++t)
    for (int n = 0; n < N; ++n)
      for (int h = 0; h < Hq; ++h) {
        const int kvh = h / nrep; /* spike_attention.py:90 */
        const int len = lens[n];
        double *o = out + (((int64_t)t * N + n) * Hq + h) * hd;
        for (int d = 0; d < hd; ++d) o[d] = 0.0;
        if (len <= 0) continue;
        const uint32_t *qw = (const uint32_t *)q + (((int64_t)t * N + n) * Hq + h) * W;
        const int64_t kvoff = ((int64_t)t * Hkv + kvh) * S;
        double *sc = (double *)malloc(sizeof(double) * len);
        double m = -INFINITY;
        for (int p = 0; p < len; ++p) {
          const int64_t slot = slot_of(tables, maxb, n, p, bs);
          const uint32_t *kw = (const uint32_t *)k + (kvoff + slot) * W;
          int cnt = 0;
          for (int w = 0; w < W; ++w) cnt += __builtin_popcount(qw[w] & kw[w]);
          sc[p] = cnt * scale;
          if (sc[p] > m) m = sc[p];
        }
        double l = 0.0;
        for (int p = 0; p < len; ++p) {
          const double e = exp(sc[p] - m);
          l += e;
          const int64_t slot = slot_of(tables, maxb, n, p, bs);
          const uint32_t *vw = (const uint32_t *)v + (kvoff + slot) * W;
          for (int d = 0; d < hd; ++d)
            if ((vw[d / 32] >> (d % 32)) & 1u) o[d] += e;
        }
        for (int d = 0; d < hd; ++d) o[d] /= l;
        free(sc);
      }
}

/* scores int32 [T, N, Hq, max_len]: popcount(q & k) for p < len, else -1. */
void orc_decode_scores(const int32_t *q, const int32_t *k, const int32_t *tables,
                       const int32_t *lens, int T, int N, int Hq, int Hkv, int hd, int bs,
                       int64_t maxb, int64_t S, int max_len, int32_t *scores) {
  const int W = (hd + 31) / 32;
  const int nrep = Hq / Hkv;
  for (int t = 0; t < T; ++t)
    for (int n = 0; n < N; ++n)
      for (int h = 0; h < Hq; ++h) {
        const uint32_t *qw = (const uint32_t *)q + (((int64_t)t * N + n) * Hq + h) * W;
        int32_t *dst = scores + (((int64_t)t * N + n) * Hq + h) * max_len;
        for (int p = 0; p < max_len; ++p) {
          if (p >= lens[n]) { dst[p] = -1; continue; }
          const int64_t slot = slot_of(tables, maxb, n, p, bs);
          const uint32_t *kw = (const uint32_t *)k + (((int64_t)t * Hkv + h / nrep) * S + slot) * W;
          int cnt = 0;
          for (int w = 0; w < W; ++w) cnt += __builtin_popcount(qw[w] & kw[w]);
          dst[p] = cnt;
        }
      }
}

/*
 * x float [T, n_tok, H, D] (contiguous); writes packed int32 words either to
 * packed [T, n_tok, H, W] (slots == NULL) or into cache [T, H, S, W] at
 * slots[i] (slots outside [0, S) skipped).
 */
void orc_lif_pack_write(const float *x, int T, int64_t n_tok, int H, int D, const float *beta,
                        const float *thr, int32_t *packed, const int64_t *slots, int64_t S) {
  const int W = (D + 31) / 32;
  const int64_t M = n_tok * H;
  uint8_t *spk = (uint8_t *)malloc((size_t)T * M * D);
  orc_lif(x, T, M, D, beta, thr, NULL, spk, NULL);
  int32_t *words = (int32_t *)malloc(sizeof(int32_t) * (size_t)T * M * W);
  orc_pack_rows(spk, (int64_t)T * M, D, words);
  for (int t = 0; t < T; ++t)
    for (int64_t i = 0; i < n_tok; ++i)
      for (int h = 0; h < H; ++h) {
        const int32_t *src = words + (((int64_t)t * n_tok + i) * H + h) * W;
        int32_t *dst;
        if (slots) {
          if (slots[i] < 0 || slots[i] >= S) continue;
          dst = packed + (((int64_t)t * H + h) * S + slots[i]) * W;
        } else {
          dst = packed + (((int64_t)t * n_tok + i) * H + h) * W;
        }
        memcpy(dst, src, sizeof(int32_t) * W);
      }
  free(words);
  free(spk);
}
