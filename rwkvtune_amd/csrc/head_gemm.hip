// LM-head GEMM for decode rows on gfx950 MFMA: logits[M, V] = A[M, K] . W^T
// with W the head weight [V][K] (bf16), fp32 accumulation, bf16 out.
//
// At decode the head is the widest projection of the step (V = 65,536 columns,
// K = 2,048 or 4,096) and M <= 128 rows, so it is bound by streaming W once
// (268 / 537 MB).  The kernel is built for that:
//   * W is packed once (head_pack_kernel) into 64-row x 32-k pieces, each a
//     contiguous 4 KB block, the pieces of one 64-row group consecutive along
//     K; a block streams its own 256 rows of W (1 MB at K = 2048) and the whole
//     activation A (L2-resident, shared by all blocks): V / 256 blocks;
//   * the block tile is BM x 256 (BM = 64 or 128) over the full K, in stages of
//     32 k filled by direct global -> LDS loads (global_load_lds_dwordx4), R
//     stages in flight; an LDS line of 128 bytes holds the 32-k slices of two
//     rows (row L and row L + BM/2, or L + 128 for W), its eight 16-byte chunks
//     at position chunk ^ swz(line), so the MFMA operand reads (32 consecutive
//     lines, one chunk each) are free of bank conflicts, as in the decode GEMM;
//   * the loop runs stage pairs with no branches: step s waits for stage s + 1,
//     issues stage s + R into the slot stage s leaves, reads stage s + 1's
//     operands into the second register set while stage s's products run; the
//     last R stages are unrolled at compile time with their own wait counts;
//   * the epilogue pairs neighbouring columns across lanes (one DPP swap) and
//     stores 4 bytes per lane (16-byte chunks staged through LDS measured the
//     same or slower).
// MFMA operand layout (gfx950): lane l supplies row l%32 of A and of B, k =
// 8*(l/32) .. +7; accumulator q of lane l is C[8*(q/4) + 4*(l/32) + q%4][l%32].
#include <type_traits>

#include "common.hpp"
#include "rwkv7_hip.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 32;      // k per stage
constexpr int kPiece = 2048;  // bf16 elements of one packed 64-row x 32-k piece

// Block tile: WM x WN waves, each MS x NS MFMA tiles of 32 x 32; BN = 256; R
// LDS stages.
template <int WM_, int WN_, int MS_, int NS_, int R_>
struct HeadTile {
    static constexpr int WM = WM_, WN = WN_, MS = MS_, NS = NS_, R = R_;
    static constexpr int NWAVE = WM * WN, THREADS = 64 * NWAVE;
    static constexpr int BM = 32 * MS * WM, BN = 32 * NS * WN;
    static constexpr int LINES = (BM + BN) / 2;  // 128-byte LDS lines per stage
    static constexpr int STAGE = LINES * 128;
    // direct loads (8 lines each) per wave per stage: LA of A, then LB of W
    static constexpr int LA = BM / 2 / 8 / NWAVE, LB = BN / 2 / 8 / NWAVE, PER = LA + LB;
    static_assert(BN == 256, "one block per 256 columns");
    static_assert(LA * 16 * NWAVE == BM && LB * 16 * NWAVE == BN, "loads split evenly over the waves");
    static_assert(R % 2 == 0 && R >= 2 && R <= 6, "stage pairs in the main loop, tail unrolled up to 6");
    static_assert((R - 1) * PER < 64, "vmcnt holds at most 63 outstanding loads");
    static_assert(R * STAGE <= 160 * 1024, "LDS");
};

using TileM64 = HeadTile<1, 4, 2, 2, 6>;   // 64 x 256, 4 waves, 6 stages (120 KB)
using TileM128 = HeadTile<2, 4, 2, 2, 4>;  // 128 x 256, 8 waves, 4 stages (96 KB)

// LDS position of logical chunk c of line r (conflict-free for 32 and 64 banks)
__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }

// s_waitcnt vmcnt(N) lgkmcnt(0)
template <int N>
__device__ __forceinline__ void wait_vm_lgkm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((N >> 4) << 14));
}

// Stage s of the block into ring slot s % R: wave w's A load i fills lines
// 8 (i NWAVE + w) .. +7, its W load i the lines BM/2 + 8 (i NWAVE + w) .. +7;
// src* already hold each lane's stage-0 address.  W loads carry the
// non-temporal hint (streamed once).
template <class T>
__device__ __forceinline__ void issue_stage(uint8_t* ring, int s, int wave, const bf16_t* const (&srcA)[T::LA],
                                            const bf16_t* const (&srcB)[T::LB]) {
    uint8_t* dst = ring + (s % T::R) * T::STAGE;
#pragma unroll
    for (int i = 0; i < T::LA; ++i)
        __builtin_amdgcn_global_load_lds(srcA[i] + s * kBK, dst + 8 * (i * T::NWAVE + wave) * 128, 16, 0, 0);
#pragma unroll
    for (int i = 0; i < T::LB; ++i)
        __builtin_amdgcn_global_load_lds(srcB[i] + s * kPiece, dst + (T::BM / 2 + 8 * (i * T::NWAVE + wave)) * 128,
                                         16, 0, 2);
}

template <class T>
__global__ __launch_bounds__(T::THREADS) void head_logits_kernel(int M, int K, const bf16_t* __restrict__ A,
                                                                 int64_t lda, const bf16_t* __restrict__ Bp,
                                                                 bf16_t* __restrict__ C, int64_t ldc) {
    __shared__ __attribute__((aligned(16))) uint8_t ring[T::R * T::STAGE];
    const int n0 = blockIdx.x * T::BN;
    const int m0 = blockIdx.y * T::BM;
    const int nst = K / kBK;  // even and >= R + 2 (checked by the host)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    // Lane L of a load brings physical position L % 8 of line line0 + L / 8:
    // logical chunk lp = (L % 8) ^ swz(line), i.e. k chunk lp % 4 of row
    // line + (lp / 4) * half.  Rows past M read row M - 1 (results not stored).
    const bf16_t* srcA[T::LA];
    const bf16_t* srcB[T::LB];
#pragma unroll
    for (int i = 0; i < T::LA; ++i) {
        const int line = 8 * (i * T::NWAVE + wave) + (lane >> 3);
        const int lp = (lane & 7) ^ swz(line);
        const int row = line + (lp >> 2) * (T::BM / 2);
        srcA[i] = A + (int64_t)min(m0 + row, M - 1) * lda + 8 * (lp & 3);
    }
#pragma unroll
    for (int i = 0; i < T::LB; ++i) {
        const int l2 = 8 * (i * T::NWAVE + wave) + (lane >> 3);
        const int lp = (lane & 7) ^ swz(T::BM / 2 + l2);
        const int g = n0 + l2 + (lp >> 2) * (T::BN / 2);  // weight row
        srcB[i] = Bp + (int64_t)(g >> 6) * nst * kPiece + (g & 63) * kBK + 8 * (lp & 3);
    }

    f32x16 acc[T::MS][T::NS];
#pragma unroll
    for (int a = 0; a < T::MS; ++a)
#pragma unroll
        for (int b = 0; b < T::NS; ++b) acc[a][b] = f32x16{0.f};
    const int lr = lane & 31, hi = lane >> 5;
    const int wm = (wave / T::WN) * (32 * T::MS), wn = (wave % T::WN) * (32 * T::NS);
    // LDS byte offsets of this lane's operands within a stage, per k step of 16
    int offA[2][T::MS], offB[2][T::NS];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
        for (int a = 0; a < T::MS; ++a) {
            const int r0 = wm + 32 * a;  // a 32-row window lies within one half
            const int line = r0 % (T::BM / 2) + lr, lp = (r0 / (T::BM / 2)) * 4 + 2 * kk + hi;
            offA[kk][a] = line * 128 + ((lp ^ swz(line)) << 4);
        }
#pragma unroll
        for (int b = 0; b < T::NS; ++b) {
            const int r0 = wn + 32 * b;
            const int line = T::BM / 2 + r0 % (T::BN / 2) + lr, lp = (r0 / (T::BN / 2)) * 4 + 2 * kk + hi;
            offB[kk][b] = line * 128 + ((lp ^ swz(line)) << 4);
        }
    }
    typedef bf16x8_t OpA[2][T::MS];
    typedef bf16x8_t OpB[2][T::NS];
    auto read = [&](int s, OpA& oa, OpB& ob) {
        const uint8_t* st = ring + (s % T::R) * T::STAGE;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
            for (int a = 0; a < T::MS; ++a) oa[kk][a] = *reinterpret_cast<const bf16x8_t*>(st + offA[kk][a]);
#pragma unroll
            for (int b = 0; b < T::NS; ++b) ob[kk][b] = *reinterpret_cast<const bf16x8_t*>(st + offB[kk][b]);
        }
    };
    auto mma = [&](const OpA& oa, const OpB& ob) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int a = 0; a < T::MS; ++a)
#pragma unroll
                for (int b = 0; b < T::NS; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(oa[kk][a], ob[kk][b], acc[a][b], 0, 0, 0);
    };

    OpA a0, a1;
    OpB b0, b1;
    // prologue: stages 0 .. R-1 in flight; stage 0 landed (every wave waited for
    // its own loads, the barrier for everyone's) and read into set 0
#pragma unroll
    for (int s = 0; s < T::R; ++s) issue_stage<T>(ring, s, wave, srcA, srcB);
    wait_vm_lgkm<(T::R - 1) * T::PER>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");  // no LDS read moves above the barrier
    read(0, a0, b0);
    // Step s (stages up to s + R - 1 issued): wait for stage s + 1 and for this
    // wave's reads of stage s (lgkmcnt(0)); the barrier makes stage s + 1
    // visible and tells every wave that slot s % R is no longer read, so it
    // takes stage s + R; stage s + 1 is read into the other set while stage s's
    // products run.
    auto body = [&](int s, OpA& ca, OpB& cb, OpA& na, OpB& nb) {
        wait_vm_lgkm<(T::R - 2) * T::PER>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        issue_stage<T>(ring, s + T::R, wave, srcA, srcB);
        read(s + 1, na, nb);
        __builtin_amdgcn_sched_barrier(0);
        mma(ca, cb);
        __builtin_amdgcn_sched_barrier(0);
    };
    int s = 0;
    for (; s < nst - T::R; s += 2) {
        body(s, a0, b0, a1, b1);
        body(s + 1, a1, b1, a0, b0);
    }
    // tail: stages nst - R .. nst - 1, nothing left to issue; at step t the
    // stages after s + t + 1 still in flight are R - 2 - t
    auto tail = [&](auto t_c, OpA& ca, OpB& cb, OpA& na, OpB& nb) {
        constexpr int t = decltype(t_c)::value;
        if constexpr (t + 1 < T::R) {
            wait_vm_lgkm<(T::R - 2 - t) * T::PER>();
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            read(s + t + 1, na, nb);
        } else {
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the last stage's operands
        }
        __builtin_amdgcn_sched_barrier(0);
        mma(ca, cb);
        __builtin_amdgcn_sched_barrier(0);
    };
    tail(std::integral_constant<int, 0>(), a0, b0, a1, b1);
    tail(std::integral_constant<int, 1>(), a1, b1, a0, b0);
    if constexpr (T::R >= 4) {
        tail(std::integral_constant<int, 2>(), a0, b0, a1, b1);
        tail(std::integral_constant<int, 3>(), a1, b1, a0, b0);
    }
    if constexpr (T::R >= 6) {
        tail(std::integral_constant<int, 4>(), a0, b0, a1, b1);
        tail(std::integral_constant<int, 5>(), a1, b1, a0, b0);
    }

    // epilogue: lanes 2j and 2j + 1 hold columns 2j and 2j + 1 of the same rows;
    // one swap of a register with the neighbour lane (DPP quad_perm 1,0,3,2)
    // gives the even lane columns 2j..2j+1 of row r and the odd lane those of row
    // r + 1, so each lane stores 4 bytes
    const bool odd = lr & 1;
#pragma unroll
    for (int a = 0; a < T::MS; ++a)
#pragma unroll
        for (int b = 0; b < T::NS; ++b) {
            const int col = n0 + wn + 32 * b + (lr & ~1);
#pragma unroll
            for (int q = 0; q < 16; q += 2) {
                const uint32_t v0 = f32_to_bf16(acc[a][b][q]), v1 = f32_to_bf16(acc[a][b][q + 1]);
                const uint32_t recv = (uint32_t)__builtin_amdgcn_mov_dpp((int)(odd ? v0 : v1), 0xB1, 0xF, 0xF, false);
                const uint32_t packed = odd ? (recv | (v1 << 16)) : (v0 | (recv << 16));
                const int row = m0 + wm + 32 * a + 8 * (q >> 2) + 4 * hi + (q & 3) + (odd ? 1 : 0);
                if (row < M) *reinterpret_cast<uint32_t*>(C + (int64_t)row * ldc + col) = packed;
            }
        }
}

// W [V][K] (row stride ldw) -> [ceil(V/64)][K/32][64][32]; rows past V zero.
// Thread e moves 16 bytes: chunk e % 4 of row (e / 4) % 64 of piece e / 256.
__global__ __launch_bounds__(256) void head_pack_kernel(const bf16_t* __restrict__ W, int64_t ldw, int V, int K,
                                                        bf16_t* __restrict__ out, int64_t chunks) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= chunks) return;
    const int c = (int)(e & 3), r = (int)((e >> 2) & 63);
    const int64_t piece = e >> 8;
    const int kt = (int)(piece % (K / kBK));
    const int64_t grp = piece / (K / kBK);
    const int64_t row = grp * 64 + r;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < V) v = *reinterpret_cast<const uint4*>(W + row * ldw + kt * kBK + 8 * c);
    *reinterpret_cast<uint4*>(out + e * 8) = v;
}

template <class T>
hipError_t launch_tile(int M, int V, int K, const void* A, int64_t lda, const void* Bp, void* C, int64_t ldc,
                       hipStream_t st) {
    const dim3 grid(V / T::BN, (M + T::BM - 1) / T::BM);
    hipLaunchKernelGGL(head_logits_kernel<T>, grid, dim3(T::THREADS), 0, st, M, K, (const bf16_t*)A, lda,
                       (const bf16_t*)Bp, (bf16_t*)C, ldc);
    return hipGetLastError();
}

}  // namespace

int head_min_k() { return kBK * (TileM64::R + 2); }
int head_row_tile(int M) { return M <= TileM64::BM ? TileM64::BM : TileM128::BM; }

int64_t head_packed_elems(int V, int K) { return (int64_t)((V + 63) / 64) * 64 * K; }

// Shapes are checked by the caller (capi.hip): V % 256 == 0, K % 64 == 0,
// K >= head_min_k(), 1 <= M, aligned operands.
hipError_t launch_head_logits(int M, int V, int K, const void* A, int64_t lda, const void* Bp, void* C, int64_t ldc,
                              hipStream_t st) {
    if (M <= TileM64::BM) return launch_tile<TileM64>(M, V, K, A, lda, Bp, C, ldc, st);
    return launch_tile<TileM128>(M, V, K, A, lda, Bp, C, ldc, st);
}

hipError_t launch_head_pack(const void* W, int64_t ldw, int V, int K, void* out, hipStream_t st) {
    const int64_t chunks = head_packed_elems(V, K) / 8;
    const int64_t blocks = (chunks + 255) / 256;
    hipLaunchKernelGGL(head_pack_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (const bf16_t*)W, ldw, V, K,
                       (bf16_t*)out, chunks);
    return hipGetLastError();
}
