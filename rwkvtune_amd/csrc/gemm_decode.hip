// Grouped bf16 GEMM for the decode step's projections on gfx950 MFMA.
//
// At decode the model's dense projections have M = live slots (<= 256) rows:
// r / k / v / output (C x C), the LoRA pairs (C x 64..480 and back), the FFN
// (C x 4C, 4C x C).  One launch runs up to 8 independent problems
//     C_p[M, N_p] = epi_p( act_in_p(A_p[M, K_p]) . B_p[N_p, K_p]^T )
// with B in nn.Linear layout [out][in] (row-major N x K), bf16 in, fp32
// accumulate, bf16 out.  act_in: 0 none, 1 tanh, 2 sigmoid (the activations
// between the LoRA down and up projections, model.py:211, 221); epi: 0 none,
// 1 relu(x)^2 (FFN key, model.py:337), 2 tanh, 3 sigmoid (the same LoRA
// activations applied to a down projection's output instead).
//
// At M = 256 the weights are read once per 64-row block of A and every block
// is short, so memory latency, not bandwidth or the matrix cores, bounds a
// naive tiling.  Here:
//   * a 256-thread block computes a 64 x 64 tile; each wave owns a 32 x 32
//     quadrant (v_mfma_f32_32x32x16_bf16);
//   * K is staged through LDS 64 at a time, and the global loads of the next
//     four stages are in flight in registers while one stage computes (a ring
//     of named registers: arrays indexed in loops would be placed in scratch);
//   * blocks are ordered so that the row tiles and K ranges of one column tile
//     run back to back on one XCD (blocks are dealt to the 8 XCDs round-robin),
//     where they share the weight rows through that XCD's L2;
//   * problems with too few tiles to fill the GPU split K; each range writes a
//     float32 partial tile to the caller's workspace and gemm_reduce_kernel sums
//     the ranges in order (deterministic) and applies the epilogue.
// MFMA operand layout (gfx950): lane l supplies row l%32 of A and of B, k =
// 8*(l/32) .. +7; accumulator q of lane l is C[8*(q/4) + 4*(l/32) + q%4][l%32].
#include "common.hpp"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kMaxProblems = 8;
constexpr int TM = 64, TN = 64, BK = 64;
constexpr int LS = BK + 8;             // LDS row stride (bf16), padded against bank conflicts
constexpr int RING = 4;                // stages of global loads in flight
constexpr int TILE_ELEMS = TM * TN;
constexpr int kThreads = 256;

struct GemmProblem {
    const bf16_t* A;
    const bf16_t* B;
    bf16_t* C;
    int64_t lda, ldb, ldc;
    int64_t ws_off;   // float offset of this problem's partials in the workspace
    int N, K;
    int act_in, epi;
    int block_begin;  // first block of this problem (a multiple of 8)
    int n_tiles;      // tiles along N
    int n_groups;     // ceil(n_tiles / 8)
    int splits;       // K ranges
    int k_per;        // K per range (multiple of BK)
    int red_begin;    // first block of this problem in gemm_reduce_kernel
};

struct GemmBatch {
    GemmProblem p[kMaxProblems];
    int count;
    int M;
};

__device__ __forceinline__ float act_fn(int act, float x) {
    if (act == 1) return tanhf(x);
    if (act == 2) return 1.0f / (1.0f + expf(-x));
    return x;
}

__device__ __forceinline__ uint4 apply_act8(uint4 v, int act) {
    if (act == 0) return v;
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float lo = act_fn(act, __uint_as_float(w[i] << 16));
        const float hi = act_fn(act, __uint_as_float(w[i] & 0xffff0000u));
        w[i] = (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ float epi_fn(int epi, float v) {
    if (epi == 1) {
        v = v > 0.f ? v : 0.f;
        return v * v;
    }
    if (epi == 2) return tanhf(v);
    if (epi == 3) return 1.0f / (1.0f + expf(-v));
    return v;
}

__device__ __forceinline__ uint4 sel(uint4 v, bool ok) { return ok ? v : make_uint4(0u, 0u, 0u, 0u); }

__global__ __launch_bounds__(kThreads) void gemm_decode_kernel(GemmBatch batch, float* __restrict__ ws) {
    __shared__ __attribute__((aligned(16))) bf16_t As[2][TM * LS];
    __shared__ __attribute__((aligned(16))) bf16_t Bs[2][TN * LS];

    // select the block's problem with constant indices only (a dynamic index
    // into the kernel-argument struct would copy it to scratch memory)
    const int bid = blockIdx.x;
    GemmProblem P = batch.p[0];
#pragma unroll
    for (int i = 1; i < kMaxProblems; ++i)
        if (i < batch.count && bid >= batch.p[i].block_begin) P = batch.p[i];
    const int M = batch.M;
    const int mt = (M + TM - 1) / TM;
    const int local = bid - P.block_begin;
    const int xcd = local & 7, j = local >> 3;  // block_begin is a multiple of 8: same XCD as bid
    const int per = mt * P.splits;
    const int ntile = (j / per) * 8 + xcd;
    if (ntile >= P.n_tiles) return;  // padding block of the last column group
    const int rem = j % per;
    const int mtile = rem % mt, split = rem / mt;
    const int m0 = mtile * TM, n0 = ntile * TN;
    const int kb = split * P.k_per;
    const int ke = min(P.K, kb + P.k_per);
    const int nst = (ke - kb + BK - 1) / BK;

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;

    // global -> LDS: thread t moves 16-byte chunks t and t + 256 of the A tile and
    // of the B tile per stage (64 rows x 8 chunks).  Rows past M / N read a valid
    // row (their results are not stored); chunks past the K range are zeroed.
    const int r0 = t >> 3, kq = (t & 7) * 8;     // chunk t: row r0, k offset kq; chunk t+256: row r0 + 32
    const bf16_t* a0 = P.A + (int64_t)min(m0 + r0, M - 1) * P.lda + kb + kq;
    const bf16_t* a1 = P.A + (int64_t)min(m0 + r0 + 32, M - 1) * P.lda + kb + kq;
    const bf16_t* b0 = P.B + (int64_t)min(n0 + r0, P.N - 1) * P.ldb + kb + kq;
    const bf16_t* b1 = P.B + (int64_t)min(n0 + r0 + 32, P.N - 1) * P.ldb + kb + kq;
    const int l0 = r0 * LS + kq, l1 = (r0 + 32) * LS + kq;
    const int kspan = ke - kb;

    uint4 ga0_0, ga1_0, gb0_0, gb1_0, ga0_1, ga1_1, gb0_1, gb1_1;
    uint4 ga0_2, ga1_2, gb0_2, gb1_2, ga0_3, ga1_3, gb0_3, gb1_3;
#define GD_LOAD(p, st)                                                                   \
    {                                                                                    \
        const int ko = (st) * BK;                                                        \
        const bool ok = ko + kq < kspan;                                                 \
        const int kc = ok ? ko : -kq;  /* past the range: re-read the range's first chunk */ \
        ga0_##p = sel(*reinterpret_cast<const uint4*>(a0 + kc), ok);                     \
        ga1_##p = sel(*reinterpret_cast<const uint4*>(a1 + kc), ok);                     \
        gb0_##p = sel(*reinterpret_cast<const uint4*>(b0 + kc), ok);                     \
        gb1_##p = sel(*reinterpret_cast<const uint4*>(b1 + kc), ok);                     \
    }
    GD_LOAD(0, 0)
    GD_LOAD(1, min(1, nst - 1))
    GD_LOAD(2, min(2, nst - 1))
    GD_LOAD(3, min(3, nst - 1))

    f32x16 acc = {0.f};
    const int r = lane & 31, kg = (lane >> 5) * 8;
    const int act = P.act_in;
#define GD_STEP(p)                                                                       \
    if (s0 + (p) < nst) {                                                                \
        const int s = s0 + (p);                                                          \
        const int buf = s & 1;                                                           \
        *reinterpret_cast<uint4*>(&As[buf][l0]) = apply_act8(ga0_##p, act);              \
        *reinterpret_cast<uint4*>(&As[buf][l1]) = apply_act8(ga1_##p, act);              \
        *reinterpret_cast<uint4*>(&Bs[buf][l0]) = gb0_##p;                               \
        *reinterpret_cast<uint4*>(&Bs[buf][l1]) = gb1_##p;                               \
        __syncthreads();                                                                 \
        GD_LOAD(p, min(s + RING, nst - 1))                                               \
        _Pragma("unroll") for (int kk = 0; kk < BK; kk += 16) {                          \
            const bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(&As[buf][(wm + r) * LS + kk + kg]); \
            const bf16x8_t bf = *reinterpret_cast<const bf16x8_t*>(&Bs[buf][(wn + r) * LS + kk + kg]); \
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf, acc, 0, 0, 0);         \
        }                                                                                \
    }
    // One barrier per stage: stage s writes LDS buffer s&1, which every wave
    // finished reading (stage s-2) before it reached stage s-1's barrier.
    for (int s0 = 0; s0 < nst; s0 += RING) {
        GD_STEP(0) GD_STEP(1) GD_STEP(2) GD_STEP(3)
    }
#undef GD_STEP
#undef GD_LOAD

    if (P.splits == 1) {
        const int col = n0 + wn + (lane & 31);
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int row = m0 + wm + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
            if (row < M && col < P.N) P.C[(int64_t)row * P.ldc + col] = f32_to_bf16(epi_fn(P.epi, acc[q]));
        }
        return;
    }
    // split-K: publish this range's partial tile; gemm_reduce_kernel, launched
    // next on the same stream, sums the ranges (a kernel boundary is what makes
    // another block's writes visible: the L2 of each XCD is private)
    const int tile = mtile * P.n_tiles + ntile;
    const int ntiles = mt * P.n_tiles;
    float* part = ws + P.ws_off + ((int64_t)split * ntiles + tile) * TILE_ELEMS;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const int rr = wm + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
        part[rr * TN + wn + (lane & 31)] = acc[q];
    }
}

// Sum the split-K partial tiles in split order (deterministic), apply the
// epilogue and write bf16.  One block per tile of the problems with splits > 1;
// red_begin is the problem's first block here.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmBatch batch, const float* __restrict__ ws) {
    const int bid = blockIdx.x;
    GemmProblem P = batch.p[0];
#pragma unroll
    for (int i = 1; i < kMaxProblems; ++i)
        if (i < batch.count && bid >= batch.p[i].red_begin) P = batch.p[i];
    const int tile = bid - P.red_begin;
    const int M = batch.M;
    const int mt = (M + TM - 1) / TM;
    const int ntiles = mt * P.n_tiles;
    if (P.splits <= 1 || tile >= ntiles) return;
    const int m0 = (tile / P.n_tiles) * TM, n0 = (tile % P.n_tiles) * TN;
    const float* base = ws + P.ws_off + (int64_t)tile * TILE_ELEMS;
    const int64_t stride = (int64_t)ntiles * TILE_ELEMS;
    for (int e = threadIdx.x; e < TILE_ELEMS; e += 256) {
        float v = 0.f;
        for (int s = 0; s < P.splits; ++s) v += base[s * stride + e];
        const int row = m0 + e / TN, col = n0 + e % TN;
        if (row < M && col < P.N) P.C[(int64_t)row * P.ldc + col] = f32_to_bf16(epi_fn(P.epi, v));
    }
}

// Split counts: when the launch's tiles alone would not reach ~384 blocks
// (1.5 per CU), every problem splits K into equal ranges of at least 1024 (a
// multiple of BK), at most 8; also the workspace floats and the tiles the
// reduction pass covers.
void plan(int M, int count, const int* N, const int* K, int* splits, int* k_per, int64_t* ws_floats,
          int64_t* red_tiles) {
    const int mt = (M + TM - 1) / TM;
    int64_t total = 0;
    for (int i = 0; i < count; ++i) total += (int64_t)mt * ((N[i] + TN - 1) / TN);
    const int want = (int)((384 + total - 1) / total);
    *ws_floats = 0;
    *red_tiles = 0;
    for (int i = 0; i < count; ++i) {
        const int64_t nt = (int64_t)mt * ((N[i] + TN - 1) / TN);
        int si = want;
        const int max_by_k = K[i] / 1024;
        if (si > max_by_k) si = max_by_k < 1 ? 1 : max_by_k;
        if (si > 8) si = 8;
        int kp = (K[i] + si - 1) / si;
        kp = (kp + BK - 1) / BK * BK;
        si = (K[i] + kp - 1) / kp;
        splits[i] = si;
        k_per[i] = kp;
        if (si > 1) {
            *ws_floats += (int64_t)si * nt * TILE_ELEMS;
            *red_tiles += nt;
        }
    }
}

}  // namespace

int gemm_decode_max_problems() { return kMaxProblems; }

int64_t gemm_decode_workspace(int M, int count, const int* N, const int* K) {
    int splits[kMaxProblems], k_per[kMaxProblems];
    int64_t wsf = 0, red = 0;
    plan(M, count, N, K, splits, k_per, &wsf, &red);
    return wsf;
}

// problems: count entries of {A, B, C, lda, ldb, ldc, N, K, act_in, epi}
hipError_t launch_gemm_decode(int M, int count, const void* const* A, const void* const* B, void* const* C,
                              const int64_t* lda, const int64_t* ldb, const int64_t* ldc, const int* N,
                              const int* K, const int* act_in, const int* epi, float* ws, hipStream_t st)
{
    GemmBatch b{};
    b.count = count;
    b.M = M;
    int splits[kMaxProblems], k_per[kMaxProblems];
    int64_t wsf = 0, red = 0;
    plan(M, count, N, K, splits, k_per, &wsf, &red);
    const int mt = (M + TM - 1) / TM;
    int blocks = 0, red_tiles = 0;
    int64_t ws_off = 0;
    for (int i = 0; i < count; ++i) {
        GemmProblem& p = b.p[i];
        p.A = (const bf16_t*)A[i];
        p.B = (const bf16_t*)B[i];
        p.C = (bf16_t*)C[i];
        p.lda = lda[i];
        p.ldb = ldb[i];
        p.ldc = ldc[i];
        p.N = N[i];
        p.K = K[i];
        p.act_in = act_in[i];
        p.epi = epi[i];
        p.n_tiles = (N[i] + TN - 1) / TN;
        p.n_groups = (p.n_tiles + 7) / 8;
        p.splits = splits[i];
        p.k_per = k_per[i];
        p.block_begin = blocks;
        p.ws_off = ws_off;
        p.red_begin = red_tiles;
        blocks += 8 * p.n_groups * mt * p.splits;
        const int nt = mt * p.n_tiles;
        if (p.splits > 1) {
            ws_off += (int64_t)p.splits * nt * TILE_ELEMS;
            red_tiles += nt;
        }
    }
    hipLaunchKernelGGL(gemm_decode_kernel, dim3(blocks), dim3(kThreads), 0, st, b, ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || red_tiles == 0) return e;
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3(red_tiles), dim3(256), 0, st, b, (const float*)ws);
    return hipGetLastError();
}
