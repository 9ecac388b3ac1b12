// RWKV-7 layer kernels around the WKV recurrence, for the model's stateful
// forward (rwkvtune/models/rwkv7/model.py:174-418) on gfx950.
//
// The reference runs each layer as ~45 eager torch ops.  Here the per-token
// element-wise work is fused into a handful of kernels; the dense projections
// stay library GEMMs (hipBLASLt through torch) between them:
//
//   shift_mix     residual add + (ln0) + LayerNorm + token shift + n lerps,
//                 and the x_prev state update            (model.py:196-208, 310-321, 393-409)
//   activation    tanh / sigmoid between LoRA GEMMs, relu^2 of the FFN key  (model.py:211,221,337)
//   tmix_prep     decay / a / value-residual / kk-normalise / k update: the
//                 six WKV operands of a prefill chunk     (model.py:215-227, 246-247)
//   tmix_post     GroupNorm(H) + (r*k*r_k).sum*v bonus + gate   (model.py:258-269)
//   tmix_decode   single-token fused path: prep + WKV step + post in one four-wave
//                 block per (row, head), state streamed from the slot pool
//   final_norm    residual add + ln_out on selected rows  (model.py:494)
//
// All element-wise arithmetic is fp32 (the reference rounds every op to the
// model dtype on GPU; on CPU it runs fp32, rwkvtune/inference/pipeline.py:166-175).
// Rows are token positions of a packed batch; rows of one sequence are
// contiguous.  row_slot[m] is the pool slot of row m's sequence (negative = no
// state: zero x_prev, nothing written); row_last[m] >= 0 marks the first row of a
// sequence in this call and holds the index of its last row.
#include "common.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

// Sum over the 64 lanes of a wave, returned in every lane (all lanes active).
// DPP butterflies inside each 16-lane row (lane ^1, ^2, ^7, ^15), then the four
// row sums read from lanes 0, 16, 32, 48: no LDS round trips.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_xor1(v);
    v += dpp_xor2(v);
    v += dpp_xor7(v);
    v += dpp_xor15(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

template <typename IO>
struct ResidualSrc {
    const float* x_in;      // [M, C] fp32 residual, or null when tokens/emb are used
    const IO* add;          // [M, C] branch output to add, nullable
    const int64_t* tokens;  // [M] token ids (layer 0), nullable
    const IO* emb;          // [V, C]
    int64_t vocab;
    const float* ln0_w;     // nullable: apply ln0 after the lookup / add
    const float* ln0_b;
    const float* parts;     // instead of add: float32 partial sums [n_parts][rows][C], nullable
    int n_parts;
    int64_t part_stride;    // floats between consecutive partial planes
};

// ---------------------------------------------------------------------------
// shift_mix, register-resident: thread t owns the float4 chunks t, t+256, ...
// of the row (NV chunks at most), every operand is loaded once up front, and a
// LayerNorm costs two block reductions.  Latency, not bandwidth, bounds this
// kernel at decode sizes (one row per block), so the loads are issued together.
// ---------------------------------------------------------------------------

template <typename IO> struct vec4io;
template <> struct vec4io<float> {
    static __device__ __forceinline__ f32x4 load(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
    static __device__ __forceinline__ void store(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
};
template <> struct vec4io<bf16_t> {
    static __device__ __forceinline__ f32x4 load(const bf16_t* p) { return io_traits<bf16_t>::load4(p); }
    static __device__ __forceinline__ void store(bf16_t* p, f32x4 v) {
        uint2 u;
        u.x = (uint32_t)f32_to_bf16(v.x) | ((uint32_t)f32_to_bf16(v.y) << 16);
        u.y = (uint32_t)f32_to_bf16(v.z) | ((uint32_t)f32_to_bf16(v.w) << 16);
        *reinterpret_cast<uint2*>(p) = u;
    }
};
template <> struct vec4io<f16_t> {
    static __device__ __forceinline__ f32x4 load(const f16_t* p) { return io_traits<f16_t>::load4(p); }
    static __device__ __forceinline__ void store(f16_t* p, f32x4 v) {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        h4 h;
        h.x = (_Float16)v.x; h.y = (_Float16)v.y; h.z = (_Float16)v.z; h.w = (_Float16)v.w;
        *reinterpret_cast<h4*>(p) = h;
    }
};

// the branch output added to the residual at (row, chunk c): the I/O-dtype
// tensor, or the in-order sum of the float32 partials rounded to the I/O dtype
// (what the split-K reduction would have stored)
template <typename IO>
__device__ __forceinline__ f32x4 add_term(const ResidualSrc<IO>& src, int64_t row, int C, int c) {
    if (src.parts != nullptr) {
        const f32x4 v = sum_planes(src.parts + row * C + 4 * c, src.part_stride, src.n_parts);
        if constexpr (sizeof(IO) == 4) return v;
        IO t[4];
        vec4io<IO>::store(t, v);
        return vec4io<IO>::load(t);
    }
    return vec4io<IO>::load(src.add + row * C + 4 * c);
}

// two sums over a TH-thread block at once (LDS red: 2 * TH / 64 floats)
template <int TH>
__device__ __forceinline__ f32x2 block_sum2(f32x2 v, float* red) {
    constexpr int W = TH / 64;
    v.x = wave_sum(v.x);
    v.y = wave_sum(v.y);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
        red[threadIdx.x >> 6] = v.x;
        red[W + (threadIdx.x >> 6)] = v.y;
    }
    __syncthreads();
    f32x2 s = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < W; ++i) {
        s.x += red[i];
        s.y += red[W + i];
    }
    return s;
}

template <typename IO, int NV>
struct RowRegs {
    f32x4 v[NV];
};

// residual of row m into registers (emb lookup or x_in + add)
template <typename IO, int NV, int TH>
__device__ __forceinline__ void load_row(const ResidualSrc<IO>& src, int m, int C4, RowRegs<IO, NV>& r) {
    const int t = threadIdx.x;
    if (src.tokens != nullptr) {
        const int64_t tk = src.tokens[m];
        const bool ok = tk >= 0 && tk < src.vocab;
        const IO* e = src.emb + (ok ? tk : 0) * (int64_t)C4 * 4;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int c = t + j * TH;
            f32x4 z = {0.f, 0.f, 0.f, 0.f};
            r.v[j] = (c < C4 && ok) ? vec4io<IO>::load(e + 4 * c) : z;
        }
    } else {
        const float* x = src.x_in + (size_t)m * C4 * 4;
        const bool has_add = src.add != nullptr || src.parts != nullptr;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int c = t + j * TH;
            f32x4 z = {0.f, 0.f, 0.f, 0.f};
            f32x4 a = (c < C4) ? *reinterpret_cast<const f32x4*>(x + 4 * c) : z;
            if (has_add && c < C4) a += add_term(src, m, 4 * C4, c);
            r.v[j] = a;
        }
    }
}

// in-place LayerNorm of register rows a (and b when two) with weight/bias held
// in registers (ww, bb: the row's chunks of this thread)
template <int NV, int TH>
__device__ __forceinline__ void ln_regs_pre(f32x4 (&a)[NV], f32x4 (&b)[NV], bool two, int C4, const f32x4 (&ww)[NV],
                                            const f32x4 (&bb)[NV], float* red) {
    const int t = threadIdx.x;
    const float invC = 1.0f / (float)(C4 * 4);
    f32x2 s = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if (t + j * TH < C4) {
            s.x += a[j].x + a[j].y + a[j].z + a[j].w;
            if (two) s.y += b[j].x + b[j].y + b[j].z + b[j].w;
        }
    }
    s = block_sum2<TH>(s, red);
    const float ma = s.x * invC, mb = s.y * invC;
    f32x2 q = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if (t + j * TH < C4) {
            f32x4 da = a[j] - ma;
            q.x += da.x * da.x + da.y * da.y + da.z * da.z + da.w * da.w;
            if (two) {
                f32x4 db = b[j] - mb;
                q.y += db.x * db.x + db.y * db.y + db.z * db.z + db.w * db.w;
            }
        }
    }
    q = block_sum2<TH>(q, red + 2 * (TH / 64));
    const float ia = 1.0f / sqrtf(q.x * invC + 1e-5f);
    const float ib = 1.0f / sqrtf(q.y * invC + 1e-5f);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if (t + j * TH < C4) {
            a[j] = (a[j] - ma) * ia * ww[j] + bb[j];
            if (two) b[j] = (b[j] - mb) * ib * ww[j] + bb[j];
        }
    }
}

// the same with weight/bias read from memory
template <int NV, int TH>
__device__ __forceinline__ void ln_regs(f32x4 (&a)[NV], f32x4 (&b)[NV], bool two, int C4, const float* w,
                                        const float* bv, float* red) {
    f32x4 ww[NV], bb[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = threadIdx.x + j * TH;
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        ww[j] = c < C4 ? *reinterpret_cast<const f32x4*>(w + 4 * c) : z;
        bb[j] = c < C4 ? *reinterpret_cast<const f32x4*>(bv + 4 * c) : z;
    }
    ln_regs_pre<NV, TH>(a, b, two, C4, ww, bb, red);
}

template <typename IO, int NV, int NMIX, int TH>
__global__ __launch_bounds__(TH) void shift_mix_kernel(
    int M, int C, ResidualSrc<IO> src, float* __restrict__ x_out,
    const float* __restrict__ ln_w, const float* __restrict__ ln_b,
    float* __restrict__ prev_pool, int pool_slots, const int32_t* __restrict__ row_slot,
    const int32_t* __restrict__ row_last, const float* __restrict__ mix, IO* __restrict__ out)
{
    __shared__ float red[4 * (TH / 64)];
    const int m = blockIdx.x;
    const int t = threadIdx.x;
    const int C4 = C >> 2;
    int slot = row_slot[m];
    if (slot >= pool_slots) slot = -1;
    const int last = row_last[m];
    const bool first = last >= 0 || m == 0;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};

    // embedding row of a token (null: out of range -> zero row)
    auto emb_row = [&](int row) -> const IO* {
        const int64_t tk = src.tokens[row];
        return (tk >= 0 && tk < src.vocab) ? src.emb + tk * (int64_t)C : nullptr;
    };
    const IO* e_cur = src.tokens != nullptr ? emb_row(m) : nullptr;
    const IO* e_prv = (src.tokens != nullptr && !first) ? emb_row(m - 1) : nullptr;
    // chunk c of the residual of `row` (embedding lookup, or x_in + add)
    auto resid = [&](int row, const IO* e, int c) -> f32x4 {
        if (c >= C4) return z;
        if (src.tokens != nullptr) return e != nullptr ? vec4io<IO>::load(e + 4 * c) : z;
        f32x4 a = *reinterpret_cast<const f32x4*>(src.x_in + (size_t)row * C + 4 * c);
        if (src.add != nullptr || src.parts != nullptr) a += add_term(src, row, C, c);
        return a;
    };

    // The row, the previous row (or the slot's x_prev) and the LayerNorm
    // parameters are loaded up front into plain register arrays, so their
    // latencies overlap; the mix coefficients (L2-resident) are read at use.
    // Preloading them too cost registers and blocks per CU: 7 mixes at 512
    // threads 78 instead of 60 VGPRs (three blocks per CU instead of four; 7-mix
    // launch at 256 decode rows 7.0 vs 6.8 us, at 69,568 prefill rows 785 vs 778
    // us), at 1024 threads 82 instead of 62 (one block per CU instead of two;
    // C = 4096 at 16,384 prefill rows 474 vs 408 us, at 128 decode rows 8.8 vs
    // 8.3 us).
    const float* pp = prev_pool + (size_t)(slot < 0 ? 0 : slot) * C;
    f32x4 cur[NV], prv[NV], lw[NV], lb[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = t + j * TH;
        cur[j] = resid(m, e_cur, c);
        if (first)
            prv[j] = (c < C4 && slot >= 0) ? *reinterpret_cast<const f32x4*>(pp + 4 * c) : z;
        else
            prv[j] = resid(m - 1, e_prv, c);
        lw[j] = c < C4 ? *reinterpret_cast<const f32x4*>(ln_w + 4 * c) : z;
        lb[j] = c < C4 ? *reinterpret_cast<const f32x4*>(ln_b + 4 * c) : z;
    }
    // ln0 on the residual (layer 0); the previous row needs it too
    if (src.ln0_w != nullptr) ln_regs<NV, TH>(cur, prv, !first, C4, src.ln0_w, src.ln0_b, red);
    if (x_out != nullptr) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int c = t + j * TH;
            if (c < C4) *reinterpret_cast<f32x4*>(x_out + (size_t)m * C + 4 * c) = cur[j];
        }
    }
    ln_regs_pre<NV, TH>(cur, prv, !first, C4, lw, lb, red);

#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = t + j * TH;
        if (c < C4) {
            const f32x4 x = cur[j];
            const f32x4 xx = prv[j] - x;
#pragma unroll
            for (int q = 0; q < NMIX; ++q) {
                const f32x4 mq = *reinterpret_cast<const f32x4*>(mix + (size_t)q * C + 4 * c);
                vec4io<IO>::store(out + ((size_t)q * M + m) * C + 4 * c, x + xx * mq);
            }
        }
    }
    // the new x_prev is the normalised last row of the sequence; the first
    // row's block writes it, after it has read the old value
    if (first && slot >= 0 && last >= 0 && last < M) {
        float* dst = prev_pool + (size_t)slot * C;
        if (last != m) {
            const IO* e_last = src.tokens != nullptr ? emb_row(last) : nullptr;
#pragma unroll
            for (int j = 0; j < NV; ++j) prv[j] = resid(last, e_last, t + j * TH);
            f32x4 none[NV];
#pragma unroll
            for (int j = 0; j < NV; ++j) none[j] = z;
            if (src.ln0_w != nullptr) ln_regs<NV, TH>(prv, none, false, C4, src.ln0_w, src.ln0_b, red);
            ln_regs_pre<NV, TH>(prv, none, false, C4, lw, lb, red);
#pragma unroll
            for (int j = 0; j < NV; ++j) cur[j] = prv[j];
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int c = t + j * TH;
            if (c < C4) *reinterpret_cast<f32x4*>(dst + 4 * c) = cur[j];
        }
    }
}

// y = LN_out(x_in[row] + add[row]) for the n listed rows (rows = null: 0..n-1)
template <typename IO, int NV, int TH>
__global__ __launch_bounds__(TH) void final_norm_kernel(
    int C, ResidualSrc<IO> src, const int32_t* __restrict__ rows, const float* __restrict__ ln_w,
    const float* __restrict__ ln_b, IO* __restrict__ out)
{
    __shared__ float red[4 * (TH / 64)];
    const int n = blockIdx.x;
    const int m = rows != nullptr ? rows[n] : n;
    const int C4 = C >> 2;
    RowRegs<IO, NV> row;
    load_row<IO, NV, TH>(src, m, C4, row);
    f32x4 cur[NV], none[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        cur[j] = row.v[j];
        none[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    ln_regs<NV, TH>(cur, none, false, C4, ln_w, ln_b, red);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = threadIdx.x + j * TH;
        if (c < C4) vec4io<IO>::store(out + (size_t)n * C + 4 * c, cur[j]);
    }
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// softplus as torch computes it (threshold 20: identity above)
__device__ __forceinline__ float softplusf_(float x) { return x > 20.f ? x : log1pf(expf(x)); }

__device__ __forceinline__ float activation_fn(int kind, float v) {
    if (kind == 0) return tanhf(v);
    if (kind == 1) return sigmoidf_(v);
    const float r = v > 0.f ? v : 0.f;
    return r * r;
}

// 8 consecutive elements per thread; vec: x is 16-byte aligned, so whole groups
// of 8 move with 16-byte (32-byte for float32) accesses
template <typename IO>
__global__ void activation_kernel(int kind, int64_t n, IO* __restrict__ x, int vec) {
    typedef io_traits<IO> tr;
    const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (i0 >= n) return;
    if (vec && i0 + 8 <= n) {
        if constexpr (sizeof(IO) == 2) {
            uint4 u = *reinterpret_cast<const uint4*>(x + i0);
            IO* e = reinterpret_cast<IO*>(&u);
#pragma unroll
            for (int j = 0; j < 8; ++j) e[j] = tr::from_f32(activation_fn(kind, tr::to_f32(e[j])));
            *reinterpret_cast<uint4*>(x + i0) = u;
        } else {
            f32x4 a = *reinterpret_cast<const f32x4*>(x + i0);
            f32x4 b = *reinterpret_cast<const f32x4*>(x + i0 + 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                a[j] = activation_fn(kind, a[j]);
                b[j] = activation_fn(kind, b[j]);
            }
            *reinterpret_cast<f32x4*>(x + i0) = a;
            *reinterpret_cast<f32x4*>(x + i0 + 4) = b;
        }
        return;
    }
    for (int64_t i = i0; i < n && i < i0 + 8; ++i) x[i] = tr::from_f32(activation_fn(kind, tr::to_f32(x[i])));
}

struct TmixParams {
    const float* w0; const float* a0; const float* v0;
    const float* k_k; const float* k_a; const float* r_k;
    const float* lnx_w; const float* lnx_b;
};

// Per-element pre-WKV math of one head element (lane j of the wave):
// returns the six WKV operands and the updated k / v used by the bonus term.
struct PrepOut { float w_raw, k, v, a_op, b_op; float rkr; };

template <typename IO>
__device__ __forceinline__ PrepOut tmix_prep_elem(
    int layer0, size_t off, int ch, const IO* r, const IO* k, const IO* v, const IO* wl,
    const IO* al, const IO* vl, float* vfirst, const TmixParams& P)
{
    typedef io_traits<IO> tr;
    PrepOut o;
    const float rj = tr::to_f32(r[off]);
    const float kj = tr::to_f32(k[off]);
    float vj = tr::to_f32(v[off]);
    // w = -softplus(-(w0 + w_lin)) - 0.5        (model.py:227)
    o.w_raw = -softplusf_(-(P.w0[ch] + tr::to_f32(wl[off]))) - 0.5f;
    // value residual: layer 0 records v_first, later layers mix towards it (model.py:215-218)
    if (layer0) {
        vfirst[off] = vj;
    } else {
        const float mixv = sigmoidf_(P.v0[ch] + tr::to_f32(vl[off]));
        vj = vj + (vfirst[off] - vj) * mixv;
    }
    const float aj = sigmoidf_(P.a0[ch] + tr::to_f32(al[off]));  // model.py:220
    const float kkr = kj * P.k_k[ch];                              // model.py:223
    const float nrm = sqrtf(wave_sum(kkr * kkr));
    const float kk = kkr / fmaxf(nrm, 1e-12f);                     // F.normalize, eps 1e-12
    const float kn = kj * (1.0f + (aj - 1.0f) * P.k_a[ch]);        // model.py:225
    o.k = kn;
    o.v = vj;
    o.a_op = -kk;                                                  // model.py:246
    o.b_op = kk * aj;
    o.rkr = rj * kn * P.r_k[ch];                                   // bonus term (model.py:267)
    return o;
}

// Prefill: write the six WKV operands (r, w_raw, k, v, -kk, kk*a) of every
// (row, head) in the I/O type, as the reference's model hands its WKV kernel
// tensors of the model dtype (model.py:233-247).  One wave per (row, head);
// grid (M, H/4), 256 threads.
template <typename IO>
__global__ __launch_bounds__(kThreads) void tmix_prep_kernel(
    int M, int H, int layer0, const IO* __restrict__ r, const IO* __restrict__ k,
    const IO* __restrict__ v, const IO* __restrict__ wl, const IO* __restrict__ al,
    const IO* __restrict__ vl, float* __restrict__ vfirst, TmixParams P,
    IO* __restrict__ r_op, IO* __restrict__ w_op, IO* __restrict__ k_op,
    IO* __restrict__ v_op, IO* __restrict__ a_op, IO* __restrict__ b_op)
{
    typedef io_traits<IO> tr;
    const int m = blockIdx.x;
    const int h = blockIdx.y * kWaves + (threadIdx.x >> 6);
    if (h >= H) return;  // whole wave exits together
    const int j = threadIdx.x & 63;
    const int C = H * RWKV7_HEAD;
    const int ch = h * RWKV7_HEAD + j;
    const size_t off = (size_t)m * C + ch;
    const PrepOut o = tmix_prep_elem(layer0, off, ch, r, k, v, wl, al, vl, vfirst, P);
    if (r_op != nullptr) r_op[off] = r[off];
    w_op[off] = tr::from_f32(o.w_raw);
    k_op[off] = tr::from_f32(o.k);
    v_op[off] = tr::from_f32(o.v);
    a_op[off] = tr::from_f32(o.a_op);
    b_op[off] = tr::from_f32(o.b_op);
}

__device__ __forceinline__ f32x4 ld4f(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

// Prefill prep, four channels per thread with 8-byte (16-bit I/O) or 16-byte
// (float32) accesses: 16 threads (one DPP row) per head, so the kk norm is a
// row sum.  The same math as tmix_prep_elem.  n4 = M * C / 4 threads, a
// multiple of 16; every lane stays active for the row sums.  r_op may be null
// (r is then not copied).
template <typename IO>
__global__ __launch_bounds__(kThreads) void tmix_prep4_kernel(
    int64_t n4, int C, int layer0, const IO* __restrict__ r, const IO* __restrict__ k,
    const IO* __restrict__ v, const IO* __restrict__ wl, const IO* __restrict__ al,
    const IO* __restrict__ vl, float* __restrict__ vfirst, TmixParams P,
    IO* __restrict__ r_op, IO* __restrict__ w_op, IO* __restrict__ k_op,
    IO* __restrict__ v_op, IO* __restrict__ a_op, IO* __restrict__ b_op)
{
    const int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const bool live = q < n4;
    const int64_t off = (live ? q : 0) * 4;
    const int ch = (int)(off % C);
    const f32x4 kj = vec4io<IO>::load(k + off);
    f32x4 vj = vec4io<IO>::load(v + off);
    const f32x4 wlj = vec4io<IO>::load(wl + off), alj = vec4io<IO>::load(al + off);
    const f32x4 w0 = ld4f(P.w0 + ch), a0 = ld4f(P.a0 + ch), kk_w = ld4f(P.k_k + ch), ka = ld4f(P.k_a + ch);
    f32x4 vf, vlj, v0;
    if (!layer0) {
        vf = ld4f(vfirst + off);
        vlj = vec4io<IO>::load(vl + off);
        v0 = ld4f(P.v0 + ch);
    }
    f32x4 w_raw, aj, kkr;
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        w_raw[e] = -softplusf_(-(w0[e] + wlj[e])) - 0.5f;          // model.py:227
        if (!layer0) vj[e] = vj[e] + (vf[e] - vj[e]) * sigmoidf_(v0[e] + vlj[e]);  // model.py:215-218
        aj[e] = sigmoidf_(a0[e] + alj[e]);                           // model.py:220
        kkr[e] = kj[e] * kk_w[e];                                    // model.py:223
        ss += kkr[e] * kkr[e];
    }
    const float inv = 1.0f / fmaxf(sqrtf(row16_sum(ss)), 1e-12f);  // F.normalize, eps 1e-12
    if (!live) return;
    f32x4 kn, na, nb;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float kk = kkr[e] * inv;
        kn[e] = kj[e] * (1.0f + (aj[e] - 1.0f) * ka[e]);             // model.py:225
        na[e] = -kk;                                                 // model.py:246
        nb[e] = kk * aj[e];
    }
    if (layer0) *reinterpret_cast<f32x4*>(vfirst + off) = vj;
    if (r_op != nullptr) vec4io<IO>::store(r_op + off, vec4io<IO>::load(r + off));
    vec4io<IO>::store(w_op + off, w_raw);
    vec4io<IO>::store(k_op + off, kn);
    vec4io<IO>::store(v_op + off, vj);
    vec4io<IO>::store(a_op + off, na);
    vec4io<IO>::store(b_op + off, nb);
}

// Prefill post, four channels per thread (16 per head): GroupNorm over the
// head, the bonus, the gate; the same math as tmix_post_kernel.
template <typename IO>
__global__ __launch_bounds__(kThreads) void tmix_post4_kernel(
    int64_t n4, int C, const IO* __restrict__ y, const IO* __restrict__ r_op,
    const IO* __restrict__ k_op, const IO* __restrict__ v_op, const IO* __restrict__ g,
    TmixParams P, IO* __restrict__ out)
{
    const int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const bool live = q < n4;
    const int64_t off = (live ? q : 0) * 4;
    const int ch = (int)(off % C);
    const f32x4 yj = vec4io<IO>::load(y + off), rj = vec4io<IO>::load(r_op + off);
    const f32x4 kj = vec4io<IO>::load(k_op + off), vj = vec4io<IO>::load(v_op + off);
    const f32x4 gj = vec4io<IO>::load(g + off);
    const f32x4 lw = ld4f(P.lnx_w + ch), lb = ld4f(P.lnx_b + ch), rk = ld4f(P.r_k + ch);
    const float mean = row16_sum(yj[0] + yj[1] + yj[2] + yj[3]) * (1.0f / 64.0f);
    const f32x4 d = yj - mean;
    const float var = row16_sum(d[0] * d[0] + d[1] * d[1] + d[2] * d[2] + d[3] * d[3]) * (1.0f / 64.0f);
    float bp = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) bp += rj[e] * kj[e] * rk[e];
    const float bonus = row16_sum(bp);
    if (!live) return;
    const float is = 1.0f / sqrtf(var + 64e-5f);
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = ((d[e] * is) * lw[e] + lb[e] + bonus * vj[e]) * gj[e];
    vec4io<IO>::store(out + off, o);
}

// Prefill: out = (GroupNorm_H(y) + (sum_j r_j k_j r_k_j) v) * g   (model.py:258-269)
template <typename IO>
__global__ __launch_bounds__(kThreads) void tmix_post_kernel(
    int M, int H, const IO* __restrict__ y, const IO* __restrict__ r_op,
    const IO* __restrict__ k_op, const IO* __restrict__ v_op, const IO* __restrict__ g,
    TmixParams P, IO* __restrict__ out)
{
    typedef io_traits<IO> tr;
    const int m = blockIdx.x;
    const int h = blockIdx.y * kWaves + (threadIdx.x >> 6);
    if (h >= H) return;
    const int j = threadIdx.x & 63;
    const int C = H * RWKV7_HEAD;
    const int ch = h * RWKV7_HEAD + j;
    const size_t off = (size_t)m * C + ch;
    const float yj = tr::to_f32(y[off]);
    const float mean = wave_sum(yj) * (1.0f / 64.0f);
    const float d = yj - mean;
    const float var = wave_sum(d * d) * (1.0f / 64.0f);
    const float yn = d / sqrtf(var + 64e-5f) * P.lnx_w[ch] + P.lnx_b[ch];
    const float bonus = wave_sum(tr::to_f32(r_op[off]) * tr::to_f32(k_op[off]) * P.r_k[ch]);
    out[off] = tr::from_f32((yn + bonus * tr::to_f32(v_op[off])) * tr::to_f32(g[off]));
}

// Decode: one token per row, fused prep + WKV step + post.  One 256-thread
// block per (row, head), block index = row * H + head, so consecutive blocks
// stream consecutive 16 KB states of the pool.  Wave q owns state rows
// 16q .. 16q+15 (the contiguous 4 KB [4096q, 4096q+4096) of the head's state):
// lane l = 16g + c holds S[16q + 4m + g][4c..4c+3] for m = 0..3, streamed with
// coalesced, non-temporal 128-bit accesses.  Quarter-head waves keep more state
// loads in flight per CU than one wave per head (57 against 125 VGPRs: eight
// waves per SIMD instead of four; 74% -> 75-76% of HBM peak at 256 rows x 32
// heads).  Every wave computes the element-wise prep of the head's 64 channels
// (lane l = channel l: the rows' dot products need all of them); the GroupNorm
// over the head's 64 outputs takes the waves' y through LDS and one barrier.
template <typename IO>
__global__ __launch_bounds__(256) void tmix_decode_kernel(
    int M, int H, int layer0, const IO* __restrict__ r, const IO* __restrict__ k,
    const IO* __restrict__ v, const IO* __restrict__ wl, const IO* __restrict__ al,
    const IO* __restrict__ vl, const IO* __restrict__ g, float* __restrict__ vfirst, TmixParams P,
    float* __restrict__ state, int pool_slots, const int32_t* __restrict__ row_slot,
    IO* __restrict__ out)
{
    typedef io_traits<IO> tr;
    __shared__ float sh[4][6][64];  // per wave: r, decay, k', -kk, kk*a, v of the head's channels
    __shared__ float yh[64];        // y of the head's 64 rows
    const int m = blockIdx.x / H;
    const int h = blockIdx.x - m * H;
    const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int C = H * RWKV7_HEAD;
    const size_t base = (size_t)m * C + (size_t)h * RWKV7_HEAD;
    int slot = row_slot[m];
    if (slot >= pool_slots) slot = -1;
    if (slot < 0) {  // no sequence on this row (the whole block returns)
        if (wave == 0) out[base + l] = tr::from_f32(0.f);
        return;
    }
    // state loads first, so their latency overlaps the element-wise prep
    f32x4* sp = reinterpret_cast<f32x4*>(state + ((size_t)slot * H + h) * (RWKV7_HEAD * RWKV7_HEAD)) + 256 * wave;
    f32x4 S[4];
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) S[mm] = stream_load(sp + 64 * mm + l);

    // element-wise prep, lane l = channel l of the head (wave 0 records v_first)
    const size_t off = base + l;
    const int ch = h * RWKV7_HEAD + l;
    const float rj = tr::to_f32(r[off]);
    const float kj = tr::to_f32(k[off]);
    float vj = tr::to_f32(v[off]);
    // w = -softplus(-(w0 + w_lin)) - 0.5        (model.py:227)
    const float w_raw = -softplusf_(-(P.w0[ch] + tr::to_f32(wl[off]))) - 0.5f;
    // value residual: layer 0 records v_first, later layers mix towards it (model.py:215-218)
    if (layer0) {
        if (wave == 0) vfirst[off] = vj;
    } else {
        const float mixv = sigmoidf_(P.v0[ch] + tr::to_f32(vl[off]));
        vj = vj + (vfirst[off] - vj) * mixv;
    }
    const float aj = sigmoidf_(P.a0[ch] + tr::to_f32(al[off]));  // model.py:220
    const float kkr = kj * P.k_k[ch];                              // model.py:223
    const float kk = kkr / fmaxf(sqrtf(wave_sum(kkr * kkr)), 1e-12f);  // F.normalize, eps 1e-12
    const float kn = kj * (1.0f + (aj - 1.0f) * P.k_a[ch]);        // model.py:225
    float* s = &sh[wave][0][0];
    s[0 * 64 + l] = rj;
    s[1 * 64 + l] = expf(-expf(w_raw));  // decay (wkv7s.cu:27)
    s[2 * 64 + l] = kn;
    s[3 * 64 + l] = -kk;                 // a operand (model.py:246)
    s[4 * 64 + l] = kk * aj;             // b operand
    s[5 * 64 + l] = vj;
    const float rkr = rj * kn * P.r_k[ch];  // bonus term (model.py:267)
    wave_sync();  // the exchange stays inside the wave

    const int gq = l >> 4, c = l & 15;
    const f32x4 r4 = *reinterpret_cast<const f32x4*>(&s[0 * 64 + 4 * c]);
    const f32x4 w4 = *reinterpret_cast<const f32x4*>(&s[1 * 64 + 4 * c]);
    const f32x4 k4 = *reinterpret_cast<const f32x4*>(&s[2 * 64 + 4 * c]);
    const f32x4 a4 = *reinterpret_cast<const f32x4*>(&s[3 * 64 + 4 * c]);
    const f32x4 b4 = *reinterpret_cast<const f32x4*>(&s[4 * 64 + 4 * c]);
    float yq[4];
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
        const int i = 16 * wave + 4 * mm + gq;
        const float si = row16_sum(fast_dot4(a4, S[mm]));  // sa_i
        const float vi = s[5 * 64 + i];
        f32x4 x = S[mm];
        x.x = fmaf(si, b4.x, fmaf(k4.x, vi, x.x * w4.x));
        x.y = fmaf(si, b4.y, fmaf(k4.y, vi, x.y * w4.y));
        x.z = fmaf(si, b4.z, fmaf(k4.z, vi, x.z * w4.z));
        x.w = fmaf(si, b4.w, fmaf(k4.w, vi, x.w * w4.w));
        S[mm] = x;
        yq[mm] = fast_dot4(x, r4);
    }
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) stream_store(sp + 64 * mm + l, S[mm]);
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
        const float yi = row16_sum(yq[mm]);
        if (c == 0) yh[16 * wave + 4 * mm + gq] = yi;
    }
    const float bonus = wave_sum(rkr);
    __syncthreads();
    if (wave != 0) return;
    // GroupNorm over the head (lane l = row l), bonus and gate (model.py:262-270)
    const float yl = yh[l];
    const float mean = wave_sum(yl) * (1.0f / 64.0f);
    const float d = yl - mean;
    const float var = wave_sum(d * d) * (1.0f / 64.0f);
    const float yn = d / sqrtf(var + 64e-5f) * P.lnx_w[ch] + P.lnx_b[ch];
    out[off] = tr::from_f32((yn + bonus * vj) * tr::to_f32(g[off]));
}

}  // namespace

// ---------------------------------------------------------------------------
// launchers (called from capi.hip)
// ---------------------------------------------------------------------------

template <typename IO, int NV, int TH>
static hipError_t launch_shift_mix_nv(int M, int C, const ResidualSrc<IO>& src, float* x_out, const float* ln_w,
                                      const float* ln_b, float* prev_pool, int pool_slots, const int32_t* row_slot,
                                      const int32_t* row_last, int n_mix, const float* mix, void* out, hipStream_t st)
{
    if (n_mix == 7)
        hipLaunchKernelGGL((shift_mix_kernel<IO, NV, 7, TH>), dim3(M), dim3(TH), 0, st, M, C, src, x_out, ln_w,
                           ln_b, prev_pool, pool_slots, row_slot, row_last, mix, (IO*)out);
    else if (n_mix == 6)
        hipLaunchKernelGGL((shift_mix_kernel<IO, NV, 6, TH>), dim3(M), dim3(TH), 0, st, M, C, src, x_out, ln_w,
                           ln_b, prev_pool, pool_slots, row_slot, row_last, mix, (IO*)out);
    else if (n_mix == 1)
        hipLaunchKernelGGL((shift_mix_kernel<IO, NV, 1, TH>), dim3(M), dim3(TH), 0, st, M, C, src, x_out, ln_w,
                           ln_b, prev_pool, pool_slots, row_slot, row_last, mix, (IO*)out);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// Threads per row block: one block holds a row, so wide rows get more waves
// (a CU's load rate grows with the waves issuing loads); every thread holds
// NV <= 2 float4 chunks of the row.
static int row_threads(int C) {
    const int C4 = C / 4;
    return C4 >= 1024 ? 1024 : (C4 >= 512 ? 512 : 256);
}

#define RWKV7_ROW_DISPATCH(CALL)                                   \
    {                                                              \
        const int th = row_threads(C);                             \
        const int nv = (C / 4 + th - 1) / th;                      \
        if (nv < 1 || nv > 2) return hipErrorInvalidValue;         \
        if (th == 1024) { if (nv == 1) CALL(1, 1024) else CALL(2, 1024) } \
        else if (th == 512) { if (nv == 1) CALL(1, 512) else CALL(2, 512) } \
        else { if (nv == 1) CALL(1, 256) else CALL(2, 256) }      \
    }

// n_mix in {1, 6, 7}; C a multiple of 4 and at most 8 * 1024
template <typename IO>
hipError_t launch_shift_mix(int M, int C, const float* x_in, const void* add, int add_parts, int64_t part_stride,
                            const int64_t* tokens, const void* emb, int64_t vocab, const float* ln0_w,
                            const float* ln0_b, float* x_out, const float* ln_w, const float* ln_b,
                            float* prev_pool, int pool_slots, const int32_t* row_slot, const int32_t* row_last,
                            int n_mix, const float* mix, void* out, hipStream_t st)
{
    ResidualSrc<IO> src{x_in, add_parts > 0 ? nullptr : (const IO*)add, tokens, (const IO*)emb, vocab, ln0_w,
                        ln0_b, add_parts > 0 ? (const float*)add : nullptr, add_parts, part_stride};
#define RWKV7_SM(NVV, THH) return launch_shift_mix_nv<IO, NVV, THH>(M, C, src, x_out, ln_w, ln_b, prev_pool, \
                                                                  pool_slots, row_slot, row_last, n_mix, mix, out, st);
    RWKV7_ROW_DISPATCH(RWKV7_SM)
#undef RWKV7_SM
}

template <typename IO>
hipError_t launch_final_norm(int n, int C, const float* x_in, const void* add, int add_parts, int64_t part_stride,
                             const int32_t* rows, const float* ln_w, const float* ln_b, void* out, hipStream_t st)
{
    ResidualSrc<IO> src{x_in, add_parts > 0 ? nullptr : (const IO*)add, nullptr, nullptr, 0, nullptr, nullptr,
                        add_parts > 0 ? (const float*)add : nullptr, add_parts, part_stride};
#define RWKV7_FN(NVV, THH) { hipLaunchKernelGGL((final_norm_kernel<IO, NVV, THH>), dim3(n), dim3(THH), 0, st, C, src, \
                                                rows, ln_w, ln_b, (IO*)out); return hipGetLastError(); }
    RWKV7_ROW_DISPATCH(RWKV7_FN)
#undef RWKV7_FN
}

template <typename IO>
hipError_t launch_activation(int kind, int64_t n, void* x, hipStream_t st)
{
    const unsigned grid = (unsigned)((n + 8 * 256 - 1) / (8 * 256));
    const int vec = (((uintptr_t)x) & 15) == 0;
    hipLaunchKernelGGL(activation_kernel<IO>, dim3(grid), dim3(256), 0, st, kind, n, (IO*)x, vec);
    return hipGetLastError();
}

static TmixParams make_params(const float* const* p) {
    return TmixParams{p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]};
}

template <typename IO>
bool aligned4(const void* p) { return (((uintptr_t)p) % (4 * sizeof(IO))) == 0; }

template <typename IO>
hipError_t launch_tmix_prep(int M, int H, int layer0, const void* r, const void* k, const void* v,
                            const void* wl, const void* al, const void* vl, float* vfirst,
                            const float* const* params, void* const* ops, hipStream_t st)
{
    bool vec = aligned4<IO>(r) && aligned4<IO>(k) && aligned4<IO>(v) && aligned4<IO>(wl) && aligned4<IO>(al) &&
               (layer0 || aligned4<IO>(vl)) && aligned4<float>(vfirst);
    for (int i = 0; i < 6; ++i) vec = vec && aligned4<IO>(ops[i]);
    for (int i = 0; i < 6; ++i) vec = vec && (params[i] == nullptr || aligned4<float>(params[i]));
    if (vec) {
        const int64_t n4 = (int64_t)M * H * (RWKV7_HEAD / 4);
        hipLaunchKernelGGL(tmix_prep4_kernel<IO>, dim3((unsigned)((n4 + kThreads - 1) / kThreads)), dim3(kThreads),
                           0, st, n4, H * RWKV7_HEAD, layer0, (const IO*)r, (const IO*)k, (const IO*)v,
                           (const IO*)wl, (const IO*)al, (const IO*)vl, vfirst, make_params(params), (IO*)ops[0],
                           (IO*)ops[1], (IO*)ops[2], (IO*)ops[3], (IO*)ops[4], (IO*)ops[5]);
        return hipGetLastError();
    }
    dim3 grid(M, (H + kWaves - 1) / kWaves);
    hipLaunchKernelGGL(tmix_prep_kernel<IO>, grid, dim3(kThreads), 0, st, M, H, layer0,
                       (const IO*)r, (const IO*)k, (const IO*)v, (const IO*)wl, (const IO*)al,
                       (const IO*)vl, vfirst, make_params(params), (IO*)ops[0], (IO*)ops[1], (IO*)ops[2],
                       (IO*)ops[3], (IO*)ops[4], (IO*)ops[5]);
    return hipGetLastError();
}

template <typename IO>
hipError_t launch_tmix_post(int M, int H, const void* y, const void* r_op, const void* k_op,
                            const void* v_op, const void* g, const float* const* params, void* out,
                            hipStream_t st)
{
    const bool vec = aligned4<IO>(y) && aligned4<IO>(r_op) && aligned4<IO>(k_op) && aligned4<IO>(v_op) &&
                     aligned4<IO>(g) && aligned4<IO>(out) && aligned4<float>(params[5]) &&
                     aligned4<float>(params[6]) && aligned4<float>(params[7]);
    if (vec) {
        const int64_t n4 = (int64_t)M * H * (RWKV7_HEAD / 4);
        hipLaunchKernelGGL(tmix_post4_kernel<IO>, dim3((unsigned)((n4 + kThreads - 1) / kThreads)), dim3(kThreads),
                           0, st, n4, H * RWKV7_HEAD, (const IO*)y, (const IO*)r_op, (const IO*)k_op,
                           (const IO*)v_op, (const IO*)g, make_params(params), (IO*)out);
        return hipGetLastError();
    }
    dim3 grid(M, (H + kWaves - 1) / kWaves);
    hipLaunchKernelGGL(tmix_post_kernel<IO>, grid, dim3(kThreads), 0, st, M, H, (const IO*)y, (const IO*)r_op,
                       (const IO*)k_op, (const IO*)v_op, (const IO*)g, make_params(params), (IO*)out);
    return hipGetLastError();
}

template <typename IO>
hipError_t launch_tmix_decode(int M, int H, int layer0, const void* r, const void* k, const void* v,
                              const void* wl, const void* al, const void* vl, const void* g,
                              float* vfirst, const float* const* params, float* state, int pool_slots,
                              const int32_t* row_slot, void* out, hipStream_t st)
{
    hipLaunchKernelGGL(tmix_decode_kernel<IO>, dim3((unsigned)M * (unsigned)H), dim3(256), 0, st, M, H, layer0,
                       (const IO*)r, (const IO*)k, (const IO*)v, (const IO*)wl, (const IO*)al,
                       (const IO*)vl, (const IO*)g, vfirst, make_params(params), state, pool_slots,
                       row_slot, (IO*)out);
    return hipGetLastError();
}

#define RWKV7_INST_LAYER(IO)                                                                        \
    template hipError_t launch_shift_mix<IO>(int, int, const float*, const void*, int, int64_t,    \
                                             const int64_t*, const void*, int64_t, const float*,   \
                                             const float*, float*, const float*, const float*,     \
                                             float*, int, const int32_t*, const int32_t*, int,     \
                                             const float*, void*, hipStream_t);                    \
    template hipError_t launch_final_norm<IO>(int, int, const float*, const void*, int, int64_t,   \
                                              const int32_t*, const float*, const float*, void*,   \
                                              hipStream_t);                                        \
    template hipError_t launch_activation<IO>(int, int64_t, void*, hipStream_t);                   \
    template hipError_t launch_tmix_prep<IO>(int, int, int, const void*, const void*, const void*, \
                                             const void*, const void*, const void*, float*,        \
                                             const float* const*, void* const*, hipStream_t);      \
    template hipError_t launch_tmix_post<IO>(int, int, const void*, const void*, const void*,      \
                                             const void*, const void*, const float* const*,        \
                                             void*, hipStream_t);                                  \
    template hipError_t launch_tmix_decode<IO>(int, int, int, const void*, const void*,            \
                                               const void*, const void*, const void*, const void*, \
                                               const void*, float*, const float* const*, float*,   \
                                               int, const int32_t*, void*, hipStream_t);

RWKV7_INST_LAYER(float)
RWKV7_INST_LAYER(bf16_t)
RWKV7_INST_LAYER(f16_t)
