/*
 * Independent fp64 restatement of the WKV7 recurrence, in plain C.
 * TEST INFRASTRUCTURE ONLY (the checker, never the product path).
 *
 * Follows the reference CUDA kernel rwkvtune/models/rwkv7/operators/cuda/wkv7s.cu:
 *   - decay w~ = exp(-exp(w_raw))                               (wkv7s.cu:27)
 *   - sa_i = sum_j a_j S[i][j]                                  (wkv7s.cu:33-38)
 *   - S[i][j] = S[i][j]*w~_j + k_j*v_i + sa_i*b_j               (wkv7s.cu:46)
 *   - y_i = sum_j S[i][j]*r_j                                   (wkv7s.cu:47)
 * State layout [B][H][N][N], row i = value index, column j = key index (wkv7s.cu:13).
 * Inputs [B][T][H*N] as float (already upcast from the caller's I/O type),
 * output y in double.  The state is updated in place.
 *
 * wkv7_ref_ragged runs the same recurrence per sequence over a packed
 * [total][H*N] layout split by cu_seqlens, with state slot seq_slot[s] (or s when
 * seq_slot is NULL), which is the meaning of one ragged prefill call.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

static void wkv7_ref_one(int T, int H, int N, int stride_t, double *S_seq,
                         const float *r, const float *w, const float *k,
                         const float *v, const float *a, const float *b,
                         double *y)
{
    for (int t = 0; t < T; t++) {
        for (int h = 0; h < H; h++) {
            double *S = S_seq + (size_t)h * N * N;
            size_t o = (size_t)t * stride_t + (size_t)h * N;
            for (int i = 0; i < N; i++) {
                double sa = 0.0;
                for (int j = 0; j < N; j++) sa += (double)a[o + j] * S[i * N + j];
                double vi = v[o + i];
                double yi = 0.0;
                for (int j = 0; j < N; j++) {
                    double wd = exp(-exp((double)w[o + j]));
                    double s = S[i * N + j] * wd + (double)k[o + j] * vi + sa * (double)b[o + j];
                    S[i * N + j] = s;
                    yi += s * (double)r[o + j];
                }
                y[o + i] = yi;
            }
        }
    }
}

void wkv7_ref_f64(int B, int T, int H, int N, double *state,
                  const float *r, const float *w, const float *k,
                  const float *v, const float *a, const float *b, double *y)
{
    int C = H * N;
    for (int bb = 0; bb < B; bb++) {
        size_t off = (size_t)bb * T * C;
        wkv7_ref_one(T, H, N, C, state + (size_t)bb * H * N * N,
                     r + off, w + off, k + off, v + off, a + off, b + off, y + off);
    }
}

void wkv7_ref_ragged(int nseq, const int32_t *cu_seqlens, const int32_t *seq_slot,
                     int H, int N, double *state_pool,
                     const float *r, const float *w, const float *k,
                     const float *v, const float *a, const float *b, double *y)
{
    int C = H * N;
    for (int s = 0; s < nseq; s++) {
        int lo = cu_seqlens[s], hi = cu_seqlens[s + 1];
        int slot = seq_slot ? seq_slot[s] : s;
        size_t off = (size_t)lo * C;
        wkv7_ref_one(hi - lo, H, N, C, state_pool + (size_t)slot * H * N * N,
                     r + off, w + off, k + off, v + off, a + off, b + off, y + off);
    }
}
