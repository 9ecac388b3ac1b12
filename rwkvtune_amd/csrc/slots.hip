// GPU-resident slot table for ragged continuous-batching rollout.
//
// The reference keeps this bookkeeping in Python: finished sequences leave the
// decode batch and free their slot, waiting sequences take free slots, and every
// step reads each sampled token back to the host (.item() per sequence,
// rwkvtune/inference/grpo_batch_generator.py:458-610,
// rwkvtune/inference/scheduler_core.py:250-299, 363-371, 445-511).  Here it is
// device state updated by kernels inside the decode step, so steps run back to
// back with no host round trip:
//
//   sequence table  seq_prompt[n] (index of the prefilled prompt state),
//                   seq_max_new[n], seq_ngen[n], seq_done[n],
//                   out_tok / out_logp / out_step [n, maxlen]
//   slot table      slot_seq[S] (-1 = free)
//   row table       row_slot[S] (slot of row r, or -1: what the model kernels
//                   read), tok_in[S] (next input token of row r), and with
//                   compaction slot_row[S] (row of slot s, -1 = free)
//   counters        [0] next waiting sequence, [1] finished sequences,
//                   [2] decode steps committed, [3] admissions of this step,
//                   [4] live rows (with compaction)
//   admit list      admit_slot[S], admit_src[S] for the state copy
//
// Compaction: the live slots occupy rows 0 .. live-1 (in slot order), so a step
// can run only its first rows (a multiple of a row bucket >= live) and skip the
// dead tail.  Without it (slot_row == NULL) row r is slot r.
//
// Admission takes waiting sequences in index order (sequences finished at their
// first token are skipped); a sequence's tokens depend only on its own state and
// its (sequence, position) random stream, never on which slot or row it runs in.
//
// Prefill in the slot (inline mode): a sequence may be admitted before it has a
// token (seq_ngen == 0: its prompt is prefilled into the slot afterwards).  Such
// a slot holds no row until rollout_first_kernel, given the sequence's index,
// records its first token; the next commit then gives it a row with that token
// as input, or, if the first token finished it, frees the slot for the next
// waiting sequence.
#include "common.hpp"

namespace {

enum { C_NEXT = 0, C_DONE = 1, C_STEP = 2, C_NADMIT = 3, C_LIVE = 4 };

// First generated token of every sequence (sampled from its prompt's logits), or
// with seq_idx of the n sequences seq_idx[0 .. n-1] (indices outside [0, n_seq)
// are skipped).
__global__ void rollout_first_kernel(int n, const int32_t* __restrict__ seq_idx, int n_seq, int maxlen,
                                     const int64_t* __restrict__ tok,
                                     const float* __restrict__ logp, const int32_t* __restrict__ seq_max_new,
                                     int32_t* __restrict__ seq_ngen, uint8_t* __restrict__ seq_done,
                                     int32_t* __restrict__ out_tok, float* __restrict__ out_logp,
                                     int32_t* __restrict__ out_step, int64_t eos, int first_can_finish,
                                     int32_t* __restrict__ counters)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int q = seq_idx != nullptr ? seq_idx[i] : i;
    if (q < 0 || q >= n_seq) return;
    const int64_t t = tok[i];
    out_tok[(size_t)q * maxlen] = (int32_t)t;
    out_logp[(size_t)q * maxlen] = logp[i];
    if (out_step != nullptr) out_step[(size_t)q * maxlen] = 0;
    seq_ngen[q] = 1;
    const bool fin = first_can_finish && ((eos >= 0 && t == eos) || seq_max_new[q] <= 1 || maxlen <= 1);
    seq_done[q] = fin ? 1 : 0;
    if (fin) atomicAdd(&counters[C_DONE], 1);
}

// One block of >= S threads.  Commits the step's sampled tokens (have_sample),
// retires finished sequences and admits waiting ones into free slots; then
// (slot_row non-null) ranks the live slots into rows 0 .. live-1.
__global__ __launch_bounds__(1024) void rollout_commit_kernel(
    int S, int n, int maxlen, int have_sample, const int64_t* __restrict__ tok,
    const float* __restrict__ logp, int32_t* __restrict__ slot_seq, int32_t* __restrict__ row_slot,
    int32_t* __restrict__ slot_row, int64_t* __restrict__ tok_in, const int32_t* __restrict__ seq_prompt,
    const int32_t* __restrict__ seq_max_new, int32_t* __restrict__ seq_ngen, uint8_t* __restrict__ seq_done,
    int32_t* __restrict__ out_tok, float* __restrict__ out_logp, int32_t* __restrict__ out_step, int64_t eos,
    int32_t* __restrict__ counters, int32_t* __restrict__ admit_slot, int32_t* __restrict__ admit_src)
{
    __shared__ int wave_live[16];
    const int s = threadIdx.x;
    const bool compact = slot_row != nullptr;
    if (s == 0) atomicExch(&counters[C_NADMIT], 0);
    __syncthreads();
    const int step = counters[C_STEP];
    int64_t next_tok = 0;  // the slot's next input token
    if (s < S) {
        const int q = slot_seq[s];
        const int row = compact ? slot_row[s] : s;  // the row this slot ran in
        // a free slot, or one whose sequence finished at its first token
        bool admit = q < 0 || seq_done[q];
        if (q >= 0 && !admit) {
            // the row's input, or for a slot without a row (its sequence got its
            // first token since the last commit) that token
            const int last = seq_ngen[q] - 1;
            next_tok = (row >= 0) ? tok_in[row] : (last >= 0 ? out_tok[(size_t)q * maxlen + last] : 0);
        }
        if (q >= 0 && !admit && have_sample && row >= 0) {
            const int64_t t = tok[row];
            const int pos = seq_ngen[q];
            if (pos < maxlen) {
                out_tok[(size_t)q * maxlen + pos] = (int32_t)t;
                out_logp[(size_t)q * maxlen + pos] = logp[row];
                if (out_step != nullptr) out_step[(size_t)q * maxlen + pos] = step + 1;
            }
            seq_ngen[q] = pos + 1;
            const bool fin = (eos >= 0 && t == eos) || pos + 1 >= seq_max_new[q] || pos + 1 >= maxlen;
            if (fin) {
                seq_done[q] = 1;
                atomicAdd(&counters[C_DONE], 1);
                admit = true;
            } else {
                next_tok = t;
            }
        }
        if (admit) {
            int q2;
            for (;;) {
                q2 = atomicAdd(&counters[C_NEXT], 1);
                if (q2 >= n || !seq_done[q2]) break;
            }
            if (q2 >= n) {
                slot_seq[s] = -1;
                next_tok = 0;
            } else {
                slot_seq[s] = q2;
                const int last = seq_ngen[q2] - 1;
                next_tok = out_tok[(size_t)q2 * maxlen + (last < 0 ? 0 : last)];
                const int i = atomicAdd(&counters[C_NADMIT], 1);
                admit_slot[i] = s;
                admit_src[i] = seq_prompt[q2];
            }
        }
    }
    // every thread has read its row's tok_in before any row is rewritten
    __syncthreads();
    // live: the slot's sequence has a token to feed (a sequence admitted before
    // its prefill has none yet)
    if (!compact) {
        if (s < S) {
            const int q = slot_seq[s];
            const bool live = q >= 0 && seq_ngen[q] > 0;
            row_slot[s] = live ? s : -1;
            tok_in[s] = live ? next_tok : 0;
        }
    } else {
        // rank of each live slot among the live slots: ballot within the wave,
        // wave totals through LDS
        const int q = s < S ? slot_seq[s] : -1;
        const bool live = q >= 0 && seq_ngen[q] > 0;
        const unsigned long long bal = __ballot(live);
        const int lane = s & 63, w = s >> 6;
        const int in_wave = __popcll(bal & ((1ull << lane) - 1ull));
        if (lane == 0) wave_live[w] = __popcll(bal);
        __syncthreads();
        int before = 0, total = 0;
        const int nw = (int)((blockDim.x + 63) >> 6);
        for (int i = 0; i < nw; ++i) {
            const int c = wave_live[i];
            before += i < w ? c : 0;
            total += c;
        }
        if (s < S) {
            if (live) {
                const int r = before + in_wave;
                row_slot[r] = s;
                slot_row[s] = r;
                tok_in[r] = next_tok;
            } else {
                slot_row[s] = -1;
            }
            if (s >= total) {  // rows past the live ones
                row_slot[s] = -1;
                tok_in[s] = 0;
            }
        }
        if (s == 0) counters[C_LIVE] = total;
    }
    __syncthreads();
    if (s == 0 && have_sample) counters[C_STEP] = step + 1;
}

// Per-row inputs of the sampler and the repetition penalty for this step: row r
// holds slot row_slot[r] (row_slot NULL: row r is slot r).  Its random stream is
// keyed by seq_key[q] (NULL: the sequence index q) and the sequence's position.
// seq_temp / seq_top_p / seq_top_k (nullable together): per-sequence sampling
// parameters copied to the row.
__global__ void rollout_prepare_kernel(int S, int maxlen, const int32_t* __restrict__ row_slot,
                                       const int32_t* __restrict__ slot_seq, const int64_t* __restrict__ seq_key,
                                       const int32_t* __restrict__ seq_ngen,
                                       const int32_t* __restrict__ seq_prompt,
                                       const int64_t* __restrict__ prompt_start,
                                       const int32_t* __restrict__ prompt_len, uint8_t* __restrict__ active,
                                       int64_t* __restrict__ rng_key, int32_t* __restrict__ rng_ctr,
                                       int64_t* __restrict__ hist_start, int32_t* __restrict__ hist_len,
                                       int64_t* __restrict__ hist2_start, int32_t* __restrict__ hist2_len,
                                       const float* __restrict__ seq_temp, const float* __restrict__ seq_top_p,
                                       const int32_t* __restrict__ seq_top_k, float* __restrict__ temp,
                                       float* __restrict__ top_p, int32_t* __restrict__ top_k)
{
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= S) return;
    const int s = row_slot != nullptr ? row_slot[r] : r;
    const int q = (s >= 0 && s < S) ? slot_seq[s] : -1;
    const bool on = q >= 0;
    active[r] = on ? 1 : 0;
    rng_key[r] = on ? (seq_key != nullptr ? seq_key[q] : (int64_t)q) : 0;
    rng_ctr[r] = on ? seq_ngen[q] : 0;
    if (seq_temp != nullptr && on) {
        temp[r] = seq_temp[q];
        top_p[r] = seq_top_p[q];
        top_k[r] = seq_top_k[q];
    }
    if (hist_start != nullptr) {
        const int p = on ? seq_prompt[q] : 0;
        hist_start[r] = on ? prompt_start[p] : 0;
        hist_len[r] = on ? prompt_len[p] : 0;
        hist2_start[r] = on ? (int64_t)q * maxlen : 0;
        hist2_len[r] = on ? seq_ngen[q] : 0;
    }
}

// Copy the prefilled prompt state admit_src[i] into slot admit_slot[i], every
// layer: kv [L, U|S, kv_elems], att_x / ffn_x [L, U|S, C].  Fixed grid; the
// blocks stride over the admissions counted by the commit kernel.
__global__ __launch_bounds__(256) void admit_copy_kernel(
    const int32_t* __restrict__ counters, const int32_t* __restrict__ admit_slot,
    const int32_t* __restrict__ admit_src, int L, int S, int U, int64_t kv4, int64_t c4,
    const f32x4* __restrict__ src_kv, const f32x4* __restrict__ src_ax, const f32x4* __restrict__ src_fx,
    f32x4* __restrict__ dst_kv, f32x4* __restrict__ dst_ax, f32x4* __restrict__ dst_fx)
{
    const int na = counters[C_NADMIT];
    const int64_t per = kv4 + 2 * c4;  // float4s of one (slot, layer)
    const int64_t total = (int64_t)na * L * per;
    for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < total;
         w += (int64_t)gridDim.x * blockDim.x) {
        const int64_t a = w / ((int64_t)L * per);
        const int64_t rem = w - a * (int64_t)L * per;
        const int l = (int)(rem / per);
        const int64_t e = rem - (int64_t)l * per;
        const int ds = admit_slot[a];
        const int ss = admit_src[a];
        if (ds < 0 || ds >= S || ss < 0 || ss >= U) continue;
        if (e < kv4) {
            dst_kv[((int64_t)l * S + ds) * kv4 + e] = src_kv[((int64_t)l * U + ss) * kv4 + e];
        } else if (e < kv4 + c4) {
            const int64_t c = e - kv4;
            dst_ax[((int64_t)l * S + ds) * c4 + c] = src_ax[((int64_t)l * U + ss) * c4 + c];
        } else {
            const int64_t c = e - kv4 - c4;
            dst_fx[((int64_t)l * S + ds) * c4 + c] = src_fx[((int64_t)l * U + ss) * c4 + c];
        }
    }
}

}  // namespace

hipError_t launch_rollout_first(int n, const int32_t* seq_idx, int n_seq, int maxlen, const int64_t* tok,
                                const float* logp, const int32_t* seq_max_new, int32_t* seq_ngen, uint8_t* seq_done,
                                int32_t* out_tok, float* out_logp, int32_t* out_step, int64_t eos,
                                int first_can_finish, int32_t* counters, hipStream_t st)
{
    hipLaunchKernelGGL(rollout_first_kernel, dim3((n + 255) / 256), dim3(256), 0, st, n, seq_idx, n_seq, maxlen,
                       tok, logp, seq_max_new, seq_ngen, seq_done, out_tok, out_logp, out_step, eos,
                       first_can_finish, counters);
    return hipGetLastError();
}

hipError_t launch_rollout_commit(int S, int n, int maxlen, int have_sample, const int64_t* tok, const float* logp,
                                 int32_t* slot_seq, int32_t* row_slot, int32_t* slot_row, int64_t* tok_in,
                                 const int32_t* seq_prompt,
                                 const int32_t* seq_max_new, int32_t* seq_ngen, uint8_t* seq_done,
                                 int32_t* out_tok, float* out_logp, int32_t* out_step, int64_t eos,
                                 int32_t* counters, int32_t* admit_slot, int32_t* admit_src, hipStream_t st)
{
    const int threads = ((S + 63) / 64) * 64;
    hipLaunchKernelGGL(rollout_commit_kernel, dim3(1), dim3(threads), 0, st, S, n, maxlen, have_sample, tok, logp,
                       slot_seq, row_slot, slot_row, tok_in, seq_prompt, seq_max_new, seq_ngen, seq_done, out_tok,
                       out_logp, out_step, eos, counters, admit_slot, admit_src);
    return hipGetLastError();
}

hipError_t launch_rollout_prepare(int S, int maxlen, const int32_t* row_slot, const int32_t* slot_seq,
                                  const int64_t* seq_key, const int32_t* seq_ngen,
                                  const int32_t* seq_prompt, const int64_t* prompt_start,
                                  const int32_t* prompt_len, uint8_t* active, int64_t* rng_key,
                                  int32_t* rng_ctr, int64_t* hist_start, int32_t* hist_len,
                                  int64_t* hist2_start, int32_t* hist2_len, const float* seq_temp,
                                  const float* seq_top_p, const int32_t* seq_top_k, float* temp, float* top_p,
                                  int32_t* top_k, hipStream_t st)
{
    hipLaunchKernelGGL(rollout_prepare_kernel, dim3((S + 255) / 256), dim3(256), 0, st, S, maxlen, row_slot,
                       slot_seq, seq_key, seq_ngen, seq_prompt, prompt_start, prompt_len, active, rng_key, rng_ctr, hist_start,
                       hist_len, hist2_start, hist2_len, seq_temp, seq_top_p, seq_top_k, temp, top_p, top_k);
    return hipGetLastError();
}

hipError_t launch_admit_copy(const int32_t* counters, const int32_t* admit_slot, const int32_t* admit_src, int L,
                             int S, int U, int64_t kv_elems, int64_t C, const float* src_kv, const float* src_ax,
                             const float* src_fx, float* dst_kv, float* dst_ax, float* dst_fx, hipStream_t st)
{
    hipLaunchKernelGGL(admit_copy_kernel, dim3(1024), dim3(256), 0, st, counters, admit_slot, admit_src, L, S, U,
                       kv_elems / 4, C / 4, (const f32x4*)src_kv, (const f32x4*)src_ax, (const f32x4*)src_fx,
                       (f32x4*)dst_kv, (f32x4*)dst_ax, (f32x4*)dst_fx);
    return hipGetLastError();
}
