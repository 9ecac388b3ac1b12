// Chunked WKV7 prefill on gfx950 MFMA.
//
// The reference prefills by running its token-serial kernel over each chunk
// (rwkvtune/models/rwkv7/operators/cuda/wkv7s.cu:22-53 via
// grpo_batch_generator.py:353-456): T dependent steps per (sequence, head).
// Here a chunk of L = 32 tokens is one set of dense contractions.  Per head,
// with S the [value i][key j] state at the chunk start and, per key j, the
// cumulative log-decay logD_t = sum_{u<=t} -exp(w_raw_u):
//   r~_t = r_t * D_t,  a~_t = a_t * D_{t-1},  k^_s = k_s / D_s,  b^_s = b_s / D_s,
//   kbar_s = k_s * D_L / D_s,  bbar_s = b_s * D_L / D_s
//   A_ab[s,t] = b^_s . a~_t, A_ak[s,t] = k^_s . a~_t     (s < t)
//   B_rb[s,t] = b^_s . r~_t, B_rk[s,t] = k^_s . r~_t     (s <= t)
//   SA = S a~^T + V^T A_ak + SA A_ab    (column t of SA is sa_t = S_{t-1} a_t;
//                                        A_ab strictly upper: a triangular solve)
//   Y  = S r~^T + SA B_rb + V^T B_rk    (column t is y_t)
//   S' = S diag(D_L) + SA bbar + V^T kbar
// which is the recurrence S_t = S_{t-1} (diag(w_t) + a_t b_t^T) + v_t k_t^T,
// y_t = S_t r_t (wkv7s.cu:33-48) summed in closed form over the chunk.
//
// Layout: one 256-thread block per (sequence, head) walks its chunks in order,
// the state held in LDS (~117 KB per block).  Every 16x16 output block is a
// v_mfma_f32_16x16x32_bf16 product on operands split into three bf16 parts
// (six MFMAs per step), which keeps float32-grade accuracy with the bf16
// matrix cores (a two-part split leaves ~2^-17 per product, ~5e-5 of rms on y).  The triangular solve runs on one wave (lane = value
// row).  A chunk whose per-token log-decay drops below kLogDecayFloor runs the
// exact token-serial update instead, so every input gives the recurrence's result.
#include "common.hpp"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int NH = 64;   // head size
constexpr int L = 32;    // chunk length
constexpr int SP = 68;   // padded row stride (floats) of [*][64] LDS matrices
constexpr int TP = 36;   // padded row stride (floats) of [*][32] LDS matrices
// Per-token log-decay floor of the matrix form.  32 tokens * -1.25 bound every
// scaled operand (r~, a~, k^, b^) to e^+-40, far from float overflow and from the
// denormal range, where the bf16 lo parts would lose precision.  Trained RWKV-7
// layers compute w = -softplus(..) - 0.5 (rwkvtune/models/rwkv7/model.py:147), so
// their log-decay -exp(w) >= -e^-0.5 ~ -0.61 and never reaches the fallback.
constexpr float kLogDecayFloor = -1.25f;

struct __attribute__((aligned(16))) ChunkLds {
    float S[NH][SP];                                  // state [i][j]
    float Rt[L][SP], At[L][SP], Kh[L][SP], Bh[L][SP];  // r~, a~, k^, b^ [t][j]
    float VT[NH][TP], BbT[NH][TP], KbT[NH][TP];        // v^T [i][t], bbar^T, kbar^T [j][t]
    float Aab[L][TP];                                  // [s][t]
    float AakT[L][TP], BrbT[L][TP], BrkT[L][TP];       // [t][s]
    float X[NH][TP];                                   // S a~^T + V^T A_ak, then SA  [i][t]
    float Y[NH][TP];                                   // [i][t]
    float DL[NH];                                      // D_L per key
    int slow;
};

__device__ __forceinline__ uint32_t bf16_bits(float f) { return (uint32_t)f32_to_bf16(f); }

// Split 8 consecutive floats (LDS, 16-byte aligned) into three bf16 parts
// x = p0 + p1 + p2 + e with |e| <= 2^-24 |x| (each part rounds the remaining
// residual to nearest-even; the residual subtractions are exact in fp32).
__device__ __forceinline__ void split8(const float* p, bf16x8_t& p0, bf16x8_t& p1, bf16x8_t& p2) {
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(p);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(p + 4);
    float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    uint32_t w0[4], w1[4], w2[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t part[3][2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            float rem = x[2 * q + e];
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                part[c][e] = bf16_bits(rem);
                rem -= __uint_as_float(part[c][e] << 16);
            }
        }
        w0[q] = part[0][0] | (part[0][1] << 16);
        w1[q] = part[1][0] | (part[1][1] << 16);
        w2[q] = part[2][0] | (part[2][1] << 16);
    }
    p0 = __builtin_bit_cast(bf16x8_t, make_uint4(w0[0], w0[1], w0[2], w0[3]));
    p1 = __builtin_bit_cast(bf16x8_t, make_uint4(w1[0], w1[1], w1[2], w1[3]));
    p2 = __builtin_bit_cast(bf16x8_t, make_uint4(w2[0], w2[1], w2[2], w2[3]));
}

// acc += A[16 rows][K] . B[16 rows][K]^T, rows at A + r*lda / B + r*ldb, K % 32 == 0.
// Six bf16 MFMAs per 32-wide step: every part product of order <= 2^-16
// (a0b0, a0b1, a1b0, a0b2, a1b1, a2b0), which leaves a relative error per
// product term of about 2^-24, the float32 level.  Accumulator e of lane l is
// element [4*(l/16) + e][l%16] of the block.
__device__ __forceinline__ void mma16(f32x4& acc, const float* A, int lda, const float* B, int ldb, int K,
                                     int lane) {
    const int r = lane & 15, kq = (lane >> 4) * 8;
    for (int k0 = 0; k0 < K; k0 += 32) {
        bf16x8_t a0, a1, a2, b0, b1, b2;
        split8(A + r * lda + k0 + kq, a0, a1, a2);
        split8(B + r * ldb + k0 + kq, b0, b1, b2);
        // smallest terms first
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b2, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b1, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, acc, 0, 0, 0);
    }
}

__device__ __forceinline__ f32x4 load_block(const float* C, int ldc, int lane) {
    f32x4 a;
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = C[(4 * (lane >> 4) + e) * ldc + (lane & 15)];
    return a;
}

__device__ __forceinline__ void store_block(float* C, int ldc, int lane, f32x4 a) {
#pragma unroll
    for (int e = 0; e < 4; ++e) C[(4 * (lane >> 4) + e) * ldc + (lane & 15)] = a[e];
}

// Sequence s is rows [cu_seqlens[s], cu_seqlens[s+1]) of the packed inputs, or
// [s*T_uniform, (s+1)*T_uniform) when cu_seqlens is null.
template <typename IO>
__global__ __launch_bounds__(256) void wkv7_chunk_kernel(
    int H, int T_uniform, const int32_t* __restrict__ cu_seqlens, const int32_t* __restrict__ slot_idx, int pool_slots,
    int total_tokens, float* __restrict__ state, const IO* __restrict__ r, const IO* __restrict__ w,
    const IO* __restrict__ k, const IO* __restrict__ v, const IO* __restrict__ a, const IO* __restrict__ b,
    IO* __restrict__ y)
{
    typedef io_traits<IO> tr;
    __shared__ ChunkLds sm;
    const int unit = blockIdx.x;
    const int s = unit / H;
    const int h = unit - s * H;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    const int tb = cu_seqlens != nullptr ? cu_seqlens[s] : s * T_uniform;
    const int te = cu_seqlens != nullptr ? cu_seqlens[s + 1] : tb + T_uniform;
    if (tb < 0 || te < tb || te > total_tokens || te == tb) return;  // malformed or empty: untouched
    const int slot = slot_idx != nullptr ? slot_idx[s] : s;
    if (slot < 0 || slot >= pool_slots) return;

    const int C = H * NH;
    float* gS = state + ((size_t)slot * H + h) * (NH * NH);
    for (int e = tid; e < NH * NH; e += 256) sm.S[e >> 6][e & 63] = gS[e];

    for (int t0 = tb; t0 < te; t0 += L) {
        const int n = min(L, te - t0);
        // ---- phase A: cumulative decay and scaled operands --------------------
        // thread (g, j): key / value dim j, tokens t = g, g+4, ... of the chunk
        const int g = tid >> 6;
        const int j = lane;
        if (tid == 0) sm.slow = 0;
        __syncthreads();
        float logDL = 0.f;
        bool slow = false;
        for (int t = 0; t < n; ++t) {
            const float lw = -expf(tr::to_f32(w[(size_t)(t0 + t) * C + h * NH + j]));
            slow |= !(lw >= kLogDecayFloor);
            logDL += lw;
        }
        if (slow) sm.slow = 1;  // benign race: every writer stores 1
        float logD = 0.f;        // logD_{t-1} while visiting t
        for (int t = 0; t < L; ++t) {
            const bool valid = t < n;
            const size_t off = (size_t)(t0 + (valid ? t : 0)) * C + h * NH + j;
            const float lw = valid ? -expf(tr::to_f32(w[off])) : 0.f;
            const float logDt = logD + lw;
            if ((t & 3) == g) {
                const float rt = valid ? tr::to_f32(r[off]) : 0.f;
                const float kt = valid ? tr::to_f32(k[off]) : 0.f;
                const float vt = valid ? tr::to_f32(v[off]) : 0.f;
                const float at = valid ? tr::to_f32(a[off]) : 0.f;
                const float bt = valid ? tr::to_f32(b[off]) : 0.f;
                const float Dt = expf(logDt), Dtm1 = expf(logD), iDt = expf(-logDt);
                const float ratio = expf(logDL - logDt);
                sm.Rt[t][j] = rt * Dt;
                sm.At[t][j] = at * Dtm1;
                sm.Kh[t][j] = kt * iDt;
                sm.Bh[t][j] = bt * iDt;
                sm.KbT[j][t] = kt * ratio;
                sm.BbT[j][t] = bt * ratio;
                sm.VT[j][t] = vt;
            }
            logD = logDt;
        }
        if (tid < NH) sm.DL[tid] = expf(logDL);
        __syncthreads();

        if (sm.slow) {
            // ---- exact token-serial update (any decay) -------------------------
            // thread: row i = tid / 4, columns q*16 .. q*16+15 (q = tid % 4)
            const int i = tid >> 2, q = tid & 3;
            for (int t = 0; t < n; ++t) {
                const size_t off = (size_t)(t0 + t) * C + h * NH;
                float sa = 0.f;
#pragma unroll
                for (int c = 0; c < 16; ++c) sa += tr::to_f32(a[off + q * 16 + c]) * sm.S[i][q * 16 + c];
                sa += __shfl_xor(sa, 1, 64);
                sa += __shfl_xor(sa, 2, 64);
                const float vi = tr::to_f32(v[off + i]);
                float yi = 0.f;
#pragma unroll
                for (int c = 0; c < 16; ++c) {
                    const int jj = q * 16 + c;
                    const float wd = expf(-expf(tr::to_f32(w[off + jj])));
                    const float sv = sm.S[i][jj] * wd + tr::to_f32(k[off + jj]) * vi + sa * tr::to_f32(b[off + jj]);
                    sm.S[i][jj] = sv;
                    yi += sv * tr::to_f32(r[off + jj]);
                }
                yi += __shfl_xor(yi, 1, 64);
                yi += __shfl_xor(yi, 2, 64);
                if (q == 0) y[off + i] = tr::from_f32(yi);
            }
            __syncthreads();
            continue;
        }

        // ---- phase B: L x L interaction matrices, S a~^T and S r~^T -----------
        // 32 block tasks (16x16 each), 8 per wave
        for (int task = wave; task < 32; task += 4) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            if (task < 16) {
                const int which = task >> 2, bi = (task >> 1) & 1, bj = task & 1;
                const int r0 = bi * 16, c0 = bj * 16;  // output rows / cols of the block
                float* out;
                bool strict;
                if (which == 0) {        // A_ab[s][t] = b^_s . a~_t, s < t
                    mma16(acc, &sm.Bh[r0][0], SP, &sm.At[c0][0], SP, NH, lane);
                    out = &sm.Aab[r0][c0];
                    strict = true;
                } else if (which == 1) { // A_ak^T[t][s] = a~_t . k^_s, s < t
                    mma16(acc, &sm.At[r0][0], SP, &sm.Kh[c0][0], SP, NH, lane);
                    out = &sm.AakT[r0][c0];
                    strict = true;
                } else if (which == 2) { // B_rb^T[t][s] = r~_t . b^_s, s <= t
                    mma16(acc, &sm.Rt[r0][0], SP, &sm.Bh[c0][0], SP, NH, lane);
                    out = &sm.BrbT[r0][c0];
                    strict = false;
                } else {                 // B_rk^T[t][s] = r~_t . k^_s, s <= t
                    mma16(acc, &sm.Rt[r0][0], SP, &sm.Kh[c0][0], SP, NH, lane);
                    out = &sm.BrkT[r0][c0];
                    strict = false;
                }
                // masks: A_ab keeps row < col; the transposed ones keep col < row (or <=)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int rr = r0 + 4 * (lane >> 4) + e, cc = c0 + (lane & 15);
                    bool keep;
                    if (which == 0) keep = rr < cc;
                    else keep = strict ? (cc < rr) : (cc <= rr);
                    acc[e] = keep ? acc[e] : 0.f;
                }
                store_block(out, TP, lane, acc);
            } else {
                const int t2 = task - 16;
                const int isY = t2 >> 3, bi = (t2 >> 1) & 3, bj = t2 & 1;
                const int r0 = bi * 16, c0 = bj * 16;
                if (!isY) {   // X[i][t] = S[i] . a~_t
                    mma16(acc, &sm.S[r0][0], SP, &sm.At[c0][0], SP, NH, lane);
                    store_block(&sm.X[r0][c0], TP, lane, acc);
                } else {      // Y[i][t] = S[i] . r~_t
                    mma16(acc, &sm.S[r0][0], SP, &sm.Rt[c0][0], SP, NH, lane);
                    store_block(&sm.Y[r0][c0], TP, lane, acc);
                }
            }
        }
        __syncthreads();
        // ---- phase C: X += V^T A_ak, then the triangular solve for SA ---------
        for (int task = wave; task < 8; task += 4) {
            const int bi = task >> 1, bj = task & 1;
            f32x4 acc = load_block(&sm.X[bi * 16][bj * 16], TP, lane);
            mma16(acc, &sm.VT[bi * 16][0], TP, &sm.AakT[bj * 16][0], TP, L, lane);
            store_block(&sm.X[bi * 16][bj * 16], TP, lane, acc);
        }
        __syncthreads();
        if (wave == 0) {
            // lane = value row i: sa[t] = X[i][t] + sum_{s<t} sa[s] A_ab[s][t]
            float sa[L];
#pragma unroll
            for (int t = 0; t < L; ++t) {
                float acc = sm.X[lane][t];
#pragma unroll
                for (int u = 0; u < t; ++u) acc = fmaf(sa[u], sm.Aab[u][t], acc);
                sa[t] = acc;
            }
#pragma unroll
            for (int t = 0; t < L; ++t) sm.X[lane][t] = sa[t];
        }
        __syncthreads();
        // ---- phase D: Y += SA B_rb + V^T B_rk;  S' = S D_L + SA bbar + V^T kbar
        for (int task = wave; task < 24; task += 4) {
            if (task < 8) {
                const int bi = task >> 1, bj = task & 1;
                f32x4 acc = load_block(&sm.Y[bi * 16][bj * 16], TP, lane);
                mma16(acc, &sm.X[bi * 16][0], TP, &sm.BrbT[bj * 16][0], TP, L, lane);
                mma16(acc, &sm.VT[bi * 16][0], TP, &sm.BrkT[bj * 16][0], TP, L, lane);
                store_block(&sm.Y[bi * 16][bj * 16], TP, lane, acc);
            } else {
                const int t2 = task - 8;
                const int bi = t2 >> 2, bj = t2 & 3;
                f32x4 acc;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int ii = bi * 16 + 4 * (lane >> 4) + e, jj = bj * 16 + (lane & 15);
                    acc[e] = sm.S[ii][jj] * sm.DL[jj];
                }
                mma16(acc, &sm.X[bi * 16][0], TP, &sm.BbT[bj * 16][0], TP, L, lane);
                mma16(acc, &sm.VT[bi * 16][0], TP, &sm.KbT[bj * 16][0], TP, L, lane);
                store_block(&sm.S[bi * 16][bj * 16], SP, lane, acc);
            }
        }
        __syncthreads();
        // ---- y of the chunk, coalesced along the value dim -------------------
        for (int e = tid; e < L * NH; e += 256) {
            const int t = e >> 6, i = e & 63;
            if (t < n) y[(size_t)(t0 + t) * C + h * NH + i] = tr::from_f32(sm.Y[i][t]);
        }
        __syncthreads();
    }
    for (int e = tid; e < NH * NH; e += 256) gS[e] = sm.S[e >> 6][e & 63];
}

}  // namespace

template <typename IO>
hipError_t launch_wkv7_chunk(int nseq, int H, int T_uniform, const int32_t* cu_seqlens, const int32_t* slot_idx,
                             int pool_slots, int total_tokens, float* state, const void* r, const void* w,
                             const void* k, const void* v, const void* a, const void* b, void* y, hipStream_t stream)
{
    hipLaunchKernelGGL(wkv7_chunk_kernel<IO>, dim3((unsigned)nseq * (unsigned)H), dim3(256), 0, stream, H,
                       T_uniform, cu_seqlens, slot_idx, pool_slots, total_tokens, state, (const IO*)r, (const IO*)w,
                       (const IO*)k, (const IO*)v, (const IO*)a, (const IO*)b, (IO*)y);
    return hipGetLastError();
}

template hipError_t launch_wkv7_chunk<float>(int, int, int, const int32_t*, const int32_t*, int, int, float*, const void*,
                                             const void*, const void*, const void*, const void*, const void*, void*,
                                             hipStream_t);
template hipError_t launch_wkv7_chunk<bf16_t>(int, int, int, const int32_t*, const int32_t*, int, int, float*,
                                              const void*, const void*, const void*, const void*, const void*,
                                              const void*, void*, hipStream_t);
template hipError_t launch_wkv7_chunk<f16_t>(int, int, int, const int32_t*, const int32_t*, int, int, float*, const void*,
                                             const void*, const void*, const void*, const void*, const void*, void*,
                                             hipStream_t);
