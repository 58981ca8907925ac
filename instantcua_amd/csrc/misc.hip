// Small kernels of the decode loop: greedy commit, prompt embedding, bit-exact dequantisation.
#include "icua_device.h"
#include "icua_kernels.h"

namespace icua {

// Greedy commit (Shaders.swift:1501-1571): global argmax of the lm_head partials (ties to the
// lowest id), state update, stop test, optional grammar pairs, and the embedding of the next
// token(s) into the residual rows.  One workgroup of 1024 threads.
__global__ __launch_bounds__(1024) void commit_kernel(CommitArgs a) {
    State* st = a.st;
    if (st->done) return;
    __shared__ float rv[MAXM][16];
    __shared__ int ri[MAXM][16];
    __shared__ int tok_s[MAXM];
    __shared__ int halt;
    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
    const int n = st->n;
    const bool all_rows = (st->logits_rows == n);
    const int r_first = all_rows ? 0 : n - 1;
    const int nr = max(min(n - r_first, MAXM), 0);  // rows reduced: n, or the last one
    // All rows' partials are loaded together (row indices clamped into the buffer; rows past
    // nr are reduced and discarded), then reduced per row with one barrier.
    float best[MAXM];
    int bi[MAXM];
#pragma unroll
    for (int j = 0; j < MAXM; ++j) {
        const int r = min(max(r_first + min(j, nr - 1), 0), MAXM - 1);
        best[j] = -__builtin_inff();
        bi[j] = 0x7fffffff;
        for (int i = tid; i < LMH_WAVES; i += 1024)
            argmax_merge(best[j], bi[j], a.pval[(size_t)r * LMH_WAVES + i], a.pidx[(size_t)r * LMH_WAVES + i]);
    }
#pragma unroll
    for (int j = 0; j < MAXM; ++j) {
        wave_argmax(best[j], bi[j]);
        if (lane == 0) {
            rv[j][wave] = best[j];
            ri[j][wave] = bi[j];
        }
    }
    __syncthreads();
    if (tid < nr) {
        float b2 = rv[tid][0];
        int i2 = ri[tid][0];
        for (int w = 1; w < 16; ++w) argmax_merge(b2, i2, rv[tid][w], ri[tid][w]);
        tok_s[tid] = i2;
        if (a.argmax_rows) a.argmax_rows[r_first + tid] = i2;
    }
    __syncthreads();
    const int tok_last = nr > 0 ? tok_s[nr - 1] : 0;
    if (a.verify_only) return;  // speculative verify: per-row argmax only, state untouched
    if (tid == 0) {
        halt = st->step >= st->maxsteps;  // nothing may be written past out_tokens[maxsteps + 1]
        if (halt) st->done = 1;
    }
    __syncthreads();
    if (halt) return;
    if (tid == 0) {
        int tok = tok_last;
        const bool bad = tok < 0 || tok >= VOCAB;  // no finite logit (NaN model): stop on token 0
        if (bad) tok = 0;
        st->pos += n;
        st->vis_offset = -1;
        a.out_tokens[st->step] = tok;
        st->step += 1;
        const bool grammar = st->flags & STATE_FLAG_GRAMMAR;
        const bool stop = bad || tok == st->eos0 || tok == st->eos1 || (grammar && tok == 8) || st->step >= st->maxsteps ||
                          st->pos + 2 > st->maxctx;  // no cache room for the next pass
        if (stop) {
            st->done = 1;
            st->n = 1;
            tok_s[0] = -1;
            tok_s[1] = -1;
        } else if (grammar && ((st->step == 1 && (tok == 3678 || tok == 7241 || tok == 12476 || tok == 10855 ||
                                                   tok == 11862 || tok == 1339 || tok == 1472 || tok == 24769)) ||
                               tok == 11)) {
            const int next_syntax = (tok == 11) ? 220 : 7;
            a.out_tokens[st->step] = next_syntax;
            st->step += 1;
            st->n = 2;
            tok_s[0] = tok;
            tok_s[1] = next_syntax;
        } else {
            st->n = 1;
            tok_s[0] = tok;
            tok_s[1] = -1;
        }
        st->logits_rows = 0;
    }
    __syncthreads();
    const int t0 = tok_s[0], t1 = tok_s[1];
    if (t0 < 0) return;
    for (int i = tid; i < H; i += 1024) a.x[i] = dequant_tiled(a.fmt, a.E, a.Esb, (size_t)t0, i, H);
    if (t1 >= 0)
        for (int i = tid; i < H; i += 1024) a.x[H + i] = dequant_tiled(a.fmt, a.E, a.Esb, (size_t)t1, i, H);
}

hipError_t launch_commit(const CommitArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(commit_kernel, dim3(1), dim3(1024), 0, s, a);
    return hipGetLastError();
}

// Prompt rows: token embeddings, with image-pad rows taking the visual embeddings
// (Shaders.swift:676-692).
__global__ __launch_bounds__(256) void embed_kernel(EmbedArgs a) {
    const State* st = a.st;
    if (st->done) return;
    const int t = blockIdx.x;
    if (t >= a.n) return;
    const int prow = a.row0 + t;
    int tok = a.toks[prow];
    if (tok < 0 || tok >= VOCAB) tok = 0;  // host-validated; keeps the row read inside E
    const int v = prow - st->vis_offset;
    float* xr = a.x + (size_t)t * H;
    if (a.pooler && tok == IMAGE_PAD_ID && st->vis_offset >= 0 && v >= 0 && v < st->n_vis) {
        for (int i = threadIdx.x; i < H; i += 256) xr[i] = a.pooler[(size_t)v * H + i];
    } else {
        for (int i = threadIdx.x; i < H; i += 256) xr[i] = dequant_tiled(a.fmt, a.E, a.Esb, (size_t)tok, i, H);
    }
}

hipError_t launch_embed(const EmbedArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(embed_kernel, dim3(a.n), dim3(256), 0, s, a);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void dequant_kernel(int fmt, const uint8_t* w, const uint8_t* sb, int K, int row0,
                                                       int rows, float* out, int tiled) {
    const size_t total = (size_t)rows * K;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        const size_t r = i / K;
        const int k = (int)(i % K);
        out[i] = tiled ? dequant_tiled(fmt, w, sb, (size_t)row0 + r, k, K)
                       : dequant_rowmajor(fmt, w, sb, (size_t)row0 + r, k, K);
    }
}

hipError_t launch_dequant(int fmt, const uint8_t* w, const uint8_t* sb, int K, int row0, int rows, float* out,
                          int tiled, hipStream_t s) {
    size_t total = (size_t)rows * K;
    int blocks = (int)((total + 255) / 256);
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(dequant_kernel, dim3(blocks), dim3(256), 0, s, fmt, w, sb, K, row0, rows, out, tiled);
    return hipGetLastError();
}

}  // namespace icua

namespace icua {

// Host-chosen pass geometry written on the stream (no host round trip).
__global__ void set_pass_kernel(State* st, int pos, int n, int logits_rows) {
    if (threadIdx.x == 0) {
        st->pos = pos;
        st->n = n;
        st->logits_rows = logits_rows;
    }
}

hipError_t launch_set_pass(State* st, int pos, int n, int logits_rows, hipStream_t s) {
    hipLaunchKernelGGL(set_pass_kernel, dim3(1), dim3(64), 0, s, st, pos, n, logits_rows);
    return hipGetLastError();
}

}  // namespace icua
