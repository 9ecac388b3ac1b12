// Grouped bf16 GEMM for the decode step's projections on gfx950 MFMA.
//
// At decode the model's dense projections have M = live slots (<= 256) rows:
// r / k / v / output (C x C), the LoRA pairs (C x 64..256 and back), the FFN
// (C x 4C, 4C x C) and the head (C x V).  A library GEMM call costs ~10 us at
// these sizes whatever the work, and a layer needs 14 of them; here one launch
// runs up to 8 independent problems
//     C_p[M, N_p] = act_in_p(A_p[M, K_p]) . B_p[N_p, K_p]^T      (epi_p applied to C_p)
// with B in nn.Linear layout [out][in] (row-major N x K), bf16 in, fp32
// accumulate, bf16 out.  act_in: 0 none, 1 tanh, 2 sigmoid (the activations
// between the LoRA down and up projections, model.py:211, 221); epi: 0 none,
// 1 relu(x)^2 (FFN key, model.py:337).
//
// Tiling: a 256-thread block computes a 64 x 64 tile of one problem over one
// K range; its four waves own 32 x 32 quadrants as 2 x 2 blocks of
// v_mfma_f32_16x16x32_bf16.  K is staged through LDS 128 at a time,
// double-buffered (the global loads of stage s+1 are in flight during stage s).
// MFMA operand layout (gfx950, checked on the device): lane l holds row l%16 of
// the A block and row l%16 of the B block, k = 8*(l/16) .. +7; accumulator i
// of lane l is C[4*(l/16) + i][l%16].
//
// Split-K: with M <= 256 a C x C projection has only 128 tiles, too few blocks
// to keep HBM busy, so each problem's K is cut into `splits` ranges.  Each range
// writes its float32 partial tile to the caller's workspace and a second kernel
// sums the ranges in split order (deterministic) and applies the epilogue.
#include "common.hpp"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int kMaxProblems = 8;
constexpr int TM = 64, TN = 64, TK = 128, NCH = TK / 32;
constexpr int LDS_STRIDE = TK + 8;  // bf16 elements per LDS row (padding against bank conflicts)
constexpr int TILE_ELEMS = TM * TN;

struct GemmProblem {
    const bf16_t* A;
    const bf16_t* B;
    bf16_t* C;
    int64_t lda, ldb, ldc;
    int64_t ws_off;   // float offset of this problem's partials in the workspace
    int N, K;
    int act_in, epi;
    int tile_begin;   // first block index of this problem
    int n_tiles_n;    // tiles along N
    int splits;       // K ranges
    int k_per;        // K per range (multiple of 32)
    int red_begin;    // first block of this problem in gemm_reduce_kernel
};

struct GemmBatch {
    GemmProblem p[kMaxProblems];
    int count;
    int M;
};

__device__ __forceinline__ uint4 sel(uint4 v, bool ok) { return ok ? v : make_uint4(0, 0, 0, 0); }

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
    return v;
}

__global__ __launch_bounds__(256) void gemm_decode_kernel(GemmBatch batch, float* __restrict__ ws) {
    __shared__ __align__(16) bf16_t As[2][TM * LDS_STRIDE];
    __shared__ __align__(16) bf16_t Bs[2][TN * LDS_STRIDE];

    // select the block's problem with constant indices only (a dynamic index
    // into the kernel-argument struct would copy it to scratch memory)
    const int bid = blockIdx.x;
    GemmProblem P = batch.p[0];
#pragma unroll
    for (int i = 1; i < kMaxProblems; ++i)
        if (i < batch.count && bid >= batch.p[i].tile_begin) P = batch.p[i];
    const int local = bid - P.tile_begin;
    const int split = local % P.splits;
    const int tile = local / P.splits;
    const int tn = tile % P.n_tiles_n;
    const int tm = tile / P.n_tiles_n;
    const int M = batch.M;
    const int m0 = tm * TM, n0 = tn * TN;
    const int k_beg = split * P.k_per;
    const int k_end = min(P.K, k_beg + P.k_per);
    const int nstage = (k_end - k_beg + TK - 1) / TK;

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wm = (wave >> 1) * 32;  // wave quadrant
    const int wn = (wave & 1) * 32;

    // global -> LDS: thread t moves row t/4 of the A and B tiles, k chunk
    // (t%4)*8 of each 32-wide slice of a stage (NCH slices per stage).  Rows
    // past M / N and slices past k_end are loaded from a valid address and
    // zeroed, so every load is an unconditional 16-byte global load.
    const int lr = t >> 2;
    const int lk = (t & 3) * 8;
    const bool a_ok = (m0 + lr) < M;
    const bool b_ok = (n0 + lr) < P.N;
    const bf16_t* a_row = P.A + (int64_t)(a_ok ? m0 + lr : M - 1) * P.lda + lk;
    const bf16_t* b_row = P.B + (int64_t)(b_ok ? n0 + lr : P.N - 1) * P.ldb + lk;

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    uint4 ra[NCH], rb[NCH];
    auto load_stage = [&](int s) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int k = k_beg + s * TK + 32 * c;  // start of the 32-wide slice
            const bool kv = k < k_end;
            const int ko = kv ? k : k_beg;
            ra[c] = sel(*reinterpret_cast<const uint4*>(a_row + ko), a_ok && kv);
            rb[c] = sel(*reinterpret_cast<const uint4*>(b_row + ko), b_ok && kv);
        }
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            *reinterpret_cast<uint4*>(&As[buf][lr * LDS_STRIDE + lk + 32 * c]) = apply_act8(ra[c], P.act_in);
            *reinterpret_cast<uint4*>(&Bs[buf][lr * LDS_STRIDE + lk + 32 * c]) = rb[c];
        }
    };

    if (nstage > 0) {
        load_stage(0);
        store_stage(0);
    }
    __syncthreads();
    for (int s = 0; s < nstage; ++s) {
        const int cur = s & 1;
        if (s + 1 < nstage) load_stage(s + 1);
#pragma unroll
        for (int ks = 0; ks < NCH; ++ks) {
            bf16x8_t af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = wm + i * 16 + (lane & 15);
                af[i] = *reinterpret_cast<const bf16x8_t*>(&As[cur][row * LDS_STRIDE + 32 * ks + (lane >> 4) * 8]);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int col = wn + j * 16 + (lane & 15);
                bf[j] = *reinterpret_cast<const bf16x8_t*>(&Bs[cur][col * LDS_STRIDE + 32 * ks + (lane >> 4) * 8]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (s + 1 < nstage) store_stage(cur ^ 1);
        __syncthreads();
    }

    // accumulator i of lane l is C[4*(l/16)+i][l%16] of its 16x16 block
    if (P.splits == 1) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int col = n0 + wn + j * 16 + (lane & 15);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int row = m0 + wm + i * 16 + 4 * (lane >> 4) + e;
                    if (row < M && col < P.N)
                        P.C[(int64_t)row * P.ldc + col] = f32_to_bf16(epi_fn(P.epi, acc[i][j][e]));
                }
            }
        return;
    }

    // split-K: publish this range's partial tile; gemm_reduce_kernel, launched
    // next on the same stream, sums the ranges (a kernel boundary is what makes
    // another block's writes visible: the L2 of each XCD is private)
    const int ntile = ((M + TM - 1) / TM) * P.n_tiles_n;
    float* part = ws + P.ws_off + ((int64_t)split * ntile + tile) * TILE_ELEMS;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = wm + i * 16 + 4 * (lane >> 4) + e;
                const int c = wn + j * 16 + (lane & 15);
                part[r * TN + c] = acc[i][j][e];
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
    const int ntile = ((M + TM - 1) / TM) * P.n_tiles_n;
    if (P.splits <= 1 || tile >= ntile) return;
    const int m0 = (tile / P.n_tiles_n) * TM, n0 = (tile % P.n_tiles_n) * TN;
    const float* base = ws + P.ws_off + (int64_t)tile * TILE_ELEMS;
    const int64_t stride = (int64_t)ntile * TILE_ELEMS;
    for (int e = threadIdx.x; e < TILE_ELEMS; e += 256) {
        float v = 0.f;
        for (int s = 0; s < P.splits; ++s) v += base[s * stride + e];
        const int row = m0 + e / TN, col = n0 + e % TN;
        if (row < M && col < P.N) P.C[(int64_t)row * P.ldc + col] = f32_to_bf16(epi_fn(P.epi, v));
    }
}

// Split counts per problem so that the launch has about 640 blocks, each K
// range a multiple of 32 and at least 256 wide; also the workspace floats and
// the tiles the reduction pass covers.
void plan(int M, int count, const int* N, const int* K, int* splits, int* k_per, int64_t* ws_floats,
          int64_t* red_tiles) {
    const int mt = (M + TM - 1) / TM;
    int64_t tiles = 0;
    for (int i = 0; i < count; ++i) tiles += (int64_t)mt * ((N[i] + TN - 1) / TN);
    const int64_t target = 640;
    int s = (int)((target + tiles - 1) / tiles);
    if (s < 1) s = 1;
    if (s > 16) s = 16;
    *ws_floats = 0;
    *red_tiles = 0;
    for (int i = 0; i < count; ++i) {
        int si = s;
        const int max_by_k = K[i] / 256;
        if (si > max_by_k) si = max_by_k < 1 ? 1 : max_by_k;
        int kp = (K[i] + si - 1) / si;
        kp = (kp + 31) / 32 * 32;
        si = (K[i] + kp - 1) / kp;
        splits[i] = si;
        k_per[i] = kp;
        const int64_t nt = (int64_t)mt * ((N[i] + TN - 1) / TN);
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
    int tiles = 0, red_tiles = 0;
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
        p.n_tiles_n = (N[i] + TN - 1) / TN;
        p.splits = splits[i];
        p.k_per = k_per[i];
        p.tile_begin = tiles;
        p.ws_off = ws_off;
        p.red_begin = red_tiles;
        const int nt = mt * p.n_tiles_n;
        tiles += nt * p.splits;
        if (p.splits > 1) {
            ws_off += (int64_t)p.splits * nt * TILE_ELEMS;
            red_tiles += nt;
        }
    }
    hipLaunchKernelGGL(gemm_decode_kernel, dim3(tiles), dim3(256), 0, st, b, ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || red_tiles == 0) return e;
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3(red_tiles), dim3(256), 0, st, b, (const float*)ws);
    return hipGetLastError();
}
