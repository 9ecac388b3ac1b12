// WKV7 training operator on gfx950: forward with state checkpoints and the
// backward pass ("wind backstepping"), with an optional initial state and its
// gradient for chunked infinite-context training.
//
// Reference semantics (rwkvtune/models/rwkv7/operators/cuda/wkv7_cuda.cu:10-142):
// per (sequence b, head h), zero initial state (or s0), for t = 0 .. T-1
//   sa_i = sum_j a_j S_ij                            (old state)
//   S_ij = S_ij w~_j + k_j v_i + sa_i b_j,  w~ = exp(-exp(w_raw))
//   y_i  = sum_j S_ij r_j
// The forward saves sa (float32) and the state after every 16th token and after
// the last one; the backward walks t = T-1 .. 0 carrying dS in both orientations,
// reloads S_t from the checkpoint at each segment end and steps it back one token
// at a time, S_{t-1} = (S_t - v k^T - sa b^T) diag(1 / w~) (as the reference), so
// at most 15 divisions separate any state from a stored one.  Gradients:
//   dr_i = sum_j S_t[j][i] dy_j,   dS_t += dy r^T
//   dw_i = (sum_j dS_t[j][i] S_{t-1}[j][i]) * w~_i * (-exp(w_raw_i))
//   dk_i = sum_j dS_t[j][i] v_j,   dv_i = sum_j dS_t[i][j] k_j
//   dsa_i = sum_j dS_t[i][j] b_j,  db_i = sum_j dS_t[j][i] sa_j
//   da_i = sum_j S_{t-1}[j][i] dsa_j
//   dS_{t-1}[i][j] = dS_t[i][j] w~_j + dsa_i a_j
// (the infinite-context variant, wkv7_infctx_cuda.cu:105-305, adds the incoming
// gradient of the final state and returns the initial state's gradient.)
//
// Layout (CDNA, not the reference's one-thread-per-row): a 512-thread block per
// (b, h) in the forward, two 512-thread halves in the backward (one for row i of
// the state gradient, one for column i of the state and of its gradient);
// thread (i, q) = (t / 8, t % 8) of a half holds 8 columns j = 8q .. 8q+7, so a
// sum over j is 8 FMAs (two chains) and a three-step DPP reduction over the
// row's 8 lanes, and two (forward) or four (backward) waves per SIMD hide each
// other's LDS and reduction latency.  Inputs [B, T, H, 64] in the I/O dtype move
// through LDS 16 tokens (one checkpoint segment) at a time, double-buffered: the
// next segment's global loads (8 to 16 per thread, issued together) are in
// flight while the current one computes, so the memory latency is paid once per
// segment, not once per token.
#include "common.hpp"

namespace {

constexpr int NH = 64;
constexpr int SEG = 16;  // checkpoint interval (tokens)
constexpr int TPR = 8;   // threads per state row
constexpr int JPT = NH / TPR;  // columns per thread
constexpr int TH = NH * TPR;

// sum over the 8 lanes of a row (lanes 8i .. 8i+7): quad sums, then the other quad
__device__ __forceinline__ float row_sum(float x) {
    x += dpp_xor1(x);
    x += dpp_xor2(x);
    return x + dpp_xor7(x);
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <typename IO>
__global__ __launch_bounds__(TH) void wkv7_train_fwd_kernel(
    int T, int H, const IO* __restrict__ r, const IO* __restrict__ w, const IO* __restrict__ k,
    const IO* __restrict__ v, const IO* __restrict__ a, const IO* __restrict__ b, IO* __restrict__ y,
    const float* __restrict__ s0, float* __restrict__ s_out, float* __restrict__ ckpt, float* __restrict__ sa_out)
{
    typedef io_traits<IO> tr;
    // [buffer][array][token of the segment][j]: arrays r, decay, k, a, b, v
    constexpr int NA = 6;
    __shared__ __attribute__((aligned(16))) float in[2][NA][SEG][NH];
    __shared__ __attribute__((aligned(16))) float out[2][SEG][NH];  // y, sa of the segment [t][i]
    const int bh = blockIdx.x;
    const int bb = bh / H, hh = bh - bb * H;
    const int tid = threadIdx.x;
    const int i = tid / TPR, q = tid % TPR, j0 = JPT * q;
    const int nck = (T + SEG - 1) / SEG;

    float S[JPT];
    if (s0 != nullptr) {
        const float* p = s0 + ((size_t)bh * NH + i) * NH + j0;
#pragma unroll
        for (int c = 0; c < JPT / 4; ++c) {
            const f32x4 x = *reinterpret_cast<const f32x4*>(p + 4 * c);
            S[4 * c] = x.x; S[4 * c + 1] = x.y; S[4 * c + 2] = x.z; S[4 * c + 3] = x.w;
        }
    } else {
#pragma unroll
        for (int jj = 0; jj < JPT; ++jj) S[jj] = 0.f;
    }

    // staging of a segment: flat element f = tid + TH m (m < NL) is element
    // f % 64 of token f / 64 % 16 of array f / 1024.  The loads read raw values from
    // rows clamped to T - 1 (no condition on a load, so they stay in flight together);
    // the staging turns tokens past T into zero inputs with decay 1, which leave the
    // state unchanged, so every segment runs all 16 tokens without a branch.
    constexpr int NL = NA * SEG * NH / TH;
    IO xr[NL];
    auto fetch = [&](int c) {
#pragma unroll
        for (int m = 0; m < NL; ++m) {
            const int f = tid + TH * m, arr = f >> 10, t = c * SEG + ((f >> 6) & (SEG - 1)), e = f & 63;
            const IO* sp = arr == 0 ? r : arr == 1 ? w : arr == 2 ? k : arr == 3 ? a : arr == 4 ? b : v;
            xr[m] = sp[(((size_t)bb * T + min(t, T - 1)) * H + hh) * NH + e];
        }
    };
    const int nseg = (T + SEG - 1) / SEG;
    fetch(0);
    for (int c = 0; c < nseg; ++c) {
        const int buf = c & 1;
#pragma unroll
        for (int m = 0; m < NL; ++m) {
            const int f = tid + TH * m, arr = f >> 10, u = (f >> 6) & (SEG - 1);
            const bool ok = c * SEG + u < T;
            const float x = tr::to_f32(xr[m]);
            in[buf][arr][u][f & 63] = arr == 1 ? (ok ? expf(-expf(x)) : 1.f) : (ok ? x : 0.f);
        }
        __syncthreads();
        if (c + 1 < nseg) fetch(c + 1);
        float yk[SEG / TPR], sk[SEG / TPR];  // y, sa of tokens q + 8m of the segment (this lane's row)
#pragma unroll
        for (int u = 0; u < SEG; ++u) {
            const float* rr = in[buf][0][u] + j0;
            const float* dec = in[buf][1][u] + j0;
            const float* kk = in[buf][2][u] + j0;
            const float* aa = in[buf][3][u] + j0;
            const float* bv = in[buf][4][u] + j0;
            float s1 = 0.f, s2 = 0.f;
#pragma unroll
            for (int jj = 0; jj < JPT; jj += 2) {
                s1 = fmaf(aa[jj], S[jj], s1);
                s2 = fmaf(aa[jj + 1], S[jj + 1], s2);
            }
            const float sa = row_sum(s1 + s2);
            const float vi = in[buf][5][u][i];
            float y1 = 0.f, y2 = 0.f;
#pragma unroll
            for (int jj = 0; jj < JPT; ++jj) {
                const float sv = fmaf(S[jj], dec[jj], fmaf(kk[jj], vi, sa * bv[jj]));
                S[jj] = sv;
                if (jj & 1) y2 = fmaf(sv, rr[jj], y2); else y1 = fmaf(sv, rr[jj], y1);
            }
            const float yi = row_sum(y1 + y2);
            yk[u / TPR] = q == u % TPR ? yi : yk[u / TPR];
            sk[u / TPR] = q == u % TPR ? sa : sk[u / TPR];
        }
#pragma unroll
        for (int m = 0; m < SEG / TPR; ++m) {
            out[0][q + TPR * m][i] = yk[m];
            out[1][q + TPR * m][i] = sk[m];
        }
        // the state after the segment's last token
        float* p = ckpt + (((size_t)bh * nck + c) * NH + i) * NH + j0;
#pragma unroll
        for (int cc = 0; cc < JPT / 4; ++cc)
            *reinterpret_cast<f32x4*>(p + 4 * cc) = f32x4{S[4 * cc], S[4 * cc + 1], S[4 * cc + 2], S[4 * cc + 3]};
        __syncthreads();
        // y and sa of the segment's tokens, each token's 64 rows contiguous
        const int n = min(SEG, T - c * SEG);
#pragma unroll
        for (int m = 0; m < SEG * NH / TH; ++m) {
            const int e = tid + TH * m, u = e >> 6, ii = e & 63;
            if (u < n) {
                const size_t o = (((size_t)bb * T + c * SEG + u) * H + hh) * NH + ii;
                y[o] = tr::from_f32(out[0][u][ii]);
                sa_out[o] = out[1][u][ii];
            }
        }
    }
    if (s_out != nullptr) {
        // every thread read its part of s0 at the start, so s_out may alias s0
        float* p = s_out + ((size_t)bh * NH + i) * NH + j0;
#pragma unroll
        for (int c = 0; c < JPT / 4; ++c)
            *reinterpret_cast<f32x4*>(p + 4 * c) = f32x4{S[4 * c], S[4 * c + 1], S[4 * c + 2], S[4 * c + 3]};
    }
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
// The backward runs two 512-thread halves per (sequence, head).  The row half
// carries dS[i][j] (row i of the state gradient) and produces dv and dsa; the
// column half carries S[j][i] and dS[j][i] (column i) and produces dr, dw, dk,
// db and da.  The column half needs every dsa_j of a token, which the row half
// hands over through LDS behind the token's one barrier; the row half needs
// nothing from the column half.  Thread (i, q) of a half = (t / 8, t % 8) holds
// j = 8q .. 8q+7, as in the forward; with both halves a CU runs four waves per
// SIMD, which hide the row reductions' and the barrier's latency.
constexpr int TH2 = 2 * TH;

template <typename IO>
__global__ __launch_bounds__(TH2) void wkv7_train_bwd_kernel(
    int T, int H, const IO* __restrict__ r, const IO* __restrict__ w, const IO* __restrict__ k,
    const IO* __restrict__ v, const IO* __restrict__ a, const IO* __restrict__ b, const IO* __restrict__ dy,
    const float* __restrict__ ckpt, const float* __restrict__ sa_in, const float* __restrict__ ds_in,
    IO* __restrict__ dr, IO* __restrict__ dw, IO* __restrict__ dk, IO* __restrict__ dv, IO* __restrict__ da,
    IO* __restrict__ db, float* __restrict__ ds0)
{
    typedef io_traits<IO> tr;
    // [buffer][array][token of the segment][j]: arrays r, decay, k, v, a, b, dy,
    // sa, log-decay (-exp(w_raw)), inverse decay
    constexpr int NA = 10;
    __shared__ __attribute__((aligned(16))) float in[2][NA][SEG][NH];
    __shared__ __attribute__((aligned(16))) float dsa_sh[2][NH];
    __shared__ __attribute__((aligned(16))) float gout[6][SEG][NH];  // dr, dw, dk, dv, db, da [t][i]
    const int bh = blockIdx.x;
    const int bb = bh / H, hh = bh - bb * H;
    const int tid = threadIdx.x;
    const bool col = tid >= TH;  // wave-uniform: waves 8 .. 15
    const int ht = tid & (TH - 1);
    const int i = ht / TPR, q = ht % TPR, j0 = JPT * q;
    const int nck = (T + SEG - 1) / SEG;

    // row half: dS[i][j]; column half: sT = S[j][i] and dS[j][i], for j = j0 + jj
    float sT[JPT], dS[JPT];
    if (ds_in != nullptr) {
        const float* p = ds_in + (size_t)bh * NH * NH;
#pragma unroll
        for (int jj = 0; jj < JPT; ++jj) dS[jj] = col ? p[(j0 + jj) * NH + i] : p[i * NH + j0 + jj];
    } else {
#pragma unroll
        for (int jj = 0; jj < JPT; ++jj) dS[jj] = 0.f;
    }

    // staging of a segment: flat element f = tid + TH2 m (m < NL) is element
    // f % 64 of token f / 64 % 16 of input array f / 1024 (r, w, k, v, a, b, dy,
    // sa); w also yields the log-decay and inverse-decay arrays.  Rows past T are
    // loaded clamped and staged as zero inputs with decay 1, which leave the state,
    // its gradient and every carried sum unchanged, so each segment runs all 16
    // tokens without a branch.
    constexpr int NL = 8 * SEG * NH / TH2;
    float xr[NL];
    auto fetch = [&](int c) {
#pragma unroll
        for (int m = 0; m < NL; ++m) {
            const int f = tid + TH2 * m, arr = f >> 10, t = c * SEG + ((f >> 6) & (SEG - 1)), e = f & 63;
            const size_t idx = (((size_t)bb * T + min(t, T - 1)) * H + hh) * NH + e;
            if (arr == 7) {
                xr[m] = sa_in[idx];
            } else {
                const IO* sp = arr == 0 ? r : arr == 1 ? w : arr == 2 ? k : arr == 3 ? v : arr == 4 ? a
                             : arr == 5 ? b : dy;
                xr[m] = tr::to_f32(sp[idx]);
            }
        }
    };
    float ckn[JPT];  // column half: S[j][i] after segment c (its checkpoint), loaded one segment ahead
    auto fetch_ck = [&](int c) {
        if (!col) return;
        const float* p = ckpt + ((size_t)bh * nck + c) * NH * NH;
#pragma unroll
        for (int jj = 0; jj < JPT; ++jj) ckn[jj] = p[(j0 + jj) * NH + i];
    };
    const int nseg = (T + SEG - 1) / SEG;
    fetch(nseg - 1);
    fetch_ck(nseg - 1);
    for (int c = nseg - 1; c >= 0; --c) {
        const int buf = c & 1;
#pragma unroll
        for (int m = 0; m < NL; ++m) {
            const int f = tid + TH2 * m, arr = f >> 10, u = (f >> 6) & (SEG - 1), e = f & 63;
            const bool ok = c * SEG + u < T;
            if (arr == 1) {
                const float lw = ok ? -expf(xr[m]) : 0.f;
                const float wd = expf(lw);
                in[buf][1][u][e] = wd;
                in[buf][8][u][e] = lw;
                in[buf][9][u][e] = 1.0f / wd;
            } else {
                in[buf][arr][u][e] = ok ? xr[m] : 0.f;
            }
        }
        if (col) {
#pragma unroll
            for (int jj = 0; jj < JPT; ++jj) sT[jj] = ckn[jj];
        }
        __syncthreads();
        if (c > 0) {
            fetch(c - 1);
            fetch_ck(c - 1);
        }
        // tokens q + 8m of the segment (this lane's row): column half dr, dw, dk, db,
        // da; row half dv in keep[0]
        float keep[5][SEG / TPR];
#pragma unroll
        for (int u = SEG - 1; u >= 0; --u) {
            const int par = (SEG - 1 - u) & 1;  // dsa_sh buffer of this token
            const float* rr = in[buf][0][u];
            const float* dec = in[buf][1][u];
            const float* kk = in[buf][2][u];
            const float* vv = in[buf][3][u];
            const float* aa = in[buf][4][u];
            const float* bv = in[buf][5][u];
            const float* dyv = in[buf][6][u];
            const float* sav = in[buf][7][u];
            const int ku = u / TPR;
            const bool mine = q == u % TPR;
            float gsa = 0.f;
            if (col) {
                float g1 = 0.f, g2 = 0.f;  // dr_i
#pragma unroll
                for (int jj = 0; jj < JPT; jj += 2) {
                    g1 = fmaf(sT[jj], dyv[j0 + jj], g1);
                    g2 = fmaf(sT[jj + 1], dyv[j0 + jj + 1], g2);
                }
                const float g = row_sum(g1 + g2);
                const float ri = rr[i], ki = kk[i], bi = bv[i], wi = dec[i];
                const float iwi = in[buf][9][u][i];
                float gw = 0.f, gk = 0.f, gb = 0.f;
#pragma unroll
                for (int jj = 0; jj < JPT; ++jj) {
                    const int j = j0 + jj;
                    sT[jj] = (sT[jj] - ki * vv[j] - bi * sav[j]) * iwi;
                    dS[jj] = fmaf(ri, dyv[j], dS[jj]);
                    gw = fmaf(dS[jj], sT[jj], gw);
                    gk = fmaf(dS[jj], vv[j], gk);
                    gb = fmaf(dS[jj], sav[j], gb);
                }
                gw = row_sum(gw);
                gk = row_sum(gk);
                gb = row_sum(gb);
                keep[0][ku] = mine ? g : keep[0][ku];
                keep[1][ku] = mine ? gw * wi * in[buf][8][u][i] : keep[1][ku];
                keep[2][ku] = mine ? gk : keep[2][ku];
                keep[3][ku] = mine ? gb : keep[3][ku];
            } else {
                const float dyi = dyv[i];
                float gv = 0.f;
#pragma unroll
                for (int jj = 0; jj < JPT; ++jj) {
                    const int j = j0 + jj;
                    dS[jj] = fmaf(dyi, rr[j], dS[jj]);
                    gv = fmaf(dS[jj], kk[j], gv);
                    gsa = fmaf(dS[jj], bv[j], gsa);
                }
                gv = row_sum(gv);
                gsa = row_sum(gsa);
                keep[0][ku] = mine ? gv : keep[0][ku];
                dsa_sh[par][i] = gsa;  // the row's 8 lanes store the same value
            }
            // one barrier per token: dsa_sh alternates, so the next token's write
            // goes to the other buffer, read by nobody until after this barrier
            __syncthreads();
            if (col) {
                const float* ds = dsa_sh[par];
                const float ai = aa[i], wi = dec[i];
                float a1 = 0.f, a2 = 0.f;
#pragma unroll
                for (int jj = 0; jj < JPT; jj += 2) {
                    a1 = fmaf(sT[jj], ds[j0 + jj], a1);
                    a2 = fmaf(sT[jj + 1], ds[j0 + jj + 1], a2);
                }
                const float ga = row_sum(a1 + a2);
                keep[4][ku] = mine ? ga : keep[4][ku];
#pragma unroll
                for (int jj = 0; jj < JPT; ++jj) dS[jj] = fmaf(dS[jj], wi, ai * ds[j0 + jj]);
            } else {
#pragma unroll
                for (int jj = 0; jj < JPT; ++jj) dS[jj] = fmaf(dS[jj], dec[j0 + jj], gsa * aa[j0 + jj]);
            }
        }
        if (col) {
#pragma unroll
            for (int m = 0; m < SEG / TPR; ++m) {
                gout[0][q + TPR * m][i] = keep[0][m];
                gout[1][q + TPR * m][i] = keep[1][m];
                gout[2][q + TPR * m][i] = keep[2][m];
                gout[4][q + TPR * m][i] = keep[3][m];
                gout[5][q + TPR * m][i] = keep[4][m];
            }
        } else {
#pragma unroll
            for (int m = 0; m < SEG / TPR; ++m) gout[3][q + TPR * m][i] = keep[0][m];
        }
        __syncthreads();
        // the segment's gradients, each token's 64 values contiguous
        const int n = min(SEG, T - c * SEG);
#pragma unroll
        for (int m = 0; m < SEG * NH / TH2; ++m) {
            const int e = tid + TH2 * m, u = e >> 6, ii = e & 63;
            if (u < n) {
                const size_t o = (((size_t)bb * T + c * SEG + u) * H + hh) * NH + ii;
                dr[o] = tr::from_f32(gout[0][u][ii]);
                dw[o] = tr::from_f32(gout[1][u][ii]);
                dk[o] = tr::from_f32(gout[2][u][ii]);
                dv[o] = tr::from_f32(gout[3][u][ii]);
                db[o] = tr::from_f32(gout[4][u][ii]);
                da[o] = tr::from_f32(gout[5][u][ii]);
            }
        }
    }
    if (ds0 != nullptr && !col) {
        float* p = ds0 + ((size_t)bh * NH + i) * NH + j0;
#pragma unroll
        for (int c = 0; c < JPT / 4; ++c)
            *reinterpret_cast<f32x4*>(p + 4 * c) = f32x4{dS[4 * c], dS[4 * c + 1], dS[4 * c + 2], dS[4 * c + 3]};
    }
}

}  // namespace

int64_t wkv7_train_ckpt_floats(int B, int T, int H) {
    return (int64_t)B * H * ((T + SEG - 1) / SEG) * NH * NH;
}

template <typename IO>
hipError_t launch_wkv7_train_fwd(int B, int T, int H, const void* r, const void* w, const void* k, const void* v,
                                 const void* a, const void* b, void* y, const float* s0, float* s_out, float* ckpt,
                                 float* sa, hipStream_t st)
{
    hipLaunchKernelGGL(wkv7_train_fwd_kernel<IO>, dim3((unsigned)(B * H)), dim3(TH), 0, st, T, H, (const IO*)r,
                       (const IO*)w, (const IO*)k, (const IO*)v, (const IO*)a, (const IO*)b, (IO*)y, s0, s_out, ckpt,
                       sa);
    return hipGetLastError();
}

template <typename IO>
hipError_t launch_wkv7_train_bwd(int B, int T, int H, const void* r, const void* w, const void* k, const void* v,
                                 const void* a, const void* b, const void* dy, const float* ckpt, const float* sa,
                                 const float* ds_in, void* dr, void* dw, void* dk, void* dv, void* da, void* db,
                                 float* ds0, hipStream_t st)
{
    hipLaunchKernelGGL(wkv7_train_bwd_kernel<IO>, dim3((unsigned)(B * H)), dim3(TH2), 0, st, T, H, (const IO*)r,
                       (const IO*)w, (const IO*)k, (const IO*)v, (const IO*)a, (const IO*)b, (const IO*)dy, ckpt, sa,
                       ds_in, (IO*)dr, (IO*)dw, (IO*)dk, (IO*)dv, (IO*)da, (IO*)db, ds0);
    return hipGetLastError();
}

#define RWKV7_INST_TRAIN(IO)                                                                                         \
    template hipError_t launch_wkv7_train_fwd<IO>(int, int, int, const void*, const void*, const void*, const void*, \
                                                  const void*, const void*, void*, const float*, float*, float*,   \
                                                  float*, hipStream_t);                                             \
    template hipError_t launch_wkv7_train_bwd<IO>(int, int, int, const void*, const void*, const void*, const void*, \
                                                  const void*, const void*, const void*, const float*,             \
                                                  const float*, const float*, void*, void*, void*, void*, void*,   \
                                                  void*, float*, hipStream_t);
RWKV7_INST_TRAIN(float)
RWKV7_INST_TRAIN(bf16_t)
RWKV7_INST_TRAIN(f16_t)
