// dispatch.h -- per-expert token lists from the per-token top-k (the grouping that the
// reference never materialises: its prefill routes token by token, infer.c:2190-2233).
//
// List e holds every token t with e in topk(t), in ascending t, with the top-k slot it
// came from. One block per expert scans the [T][K] assignments in order and compacts
// its matches with a ballot prefix, so the order never depends on atomics; the last
// block to finish turns the counts into offsets and packs the lists. The blocks hand
// their lists to the last one through write-through (agent-scope) stores and loads
// after their own store counts reach zero, not through __threadfence(), which would
// write back and invalidate the L2 of every XCD.
#pragma once

#include "common.h"

#define GP_TOK 32  // tokens per tile of the prefill grouped GEMMs

// One tile of a grouped GEMM: list rows [row, row + count) of expert e (e == E: the
// shared expert, whose list is every token, at rows TK + t).
struct GpTile {
    int e, row, count, pad;
};

struct DispatchArgs {
    const int *topk_idx;  // [T][K]
    int T, K, E;
    int TK;               // list rows reserved for routed pairs (Tmax * K); shared rows follow
    int routed_on, shared_on;
    GpTile *tiles;        // out: routed experts' tiles in expert order, then the shared expert's
    int *n_tiles;
    int *pair_row;        // out: [T][K] list row of (token, slot), -1 if the slot is empty
    int *tmp_tok;         // [E][T]
    int *tmp_slot;        // [E][T]
    int *counts;          // [E]
    unsigned *counter;    // zero between launches
    int *offsets;         // [E+1]
    int *tokens;          // [T*K]
    int *slots;           // [T*K]
};

#define DP_BLOCK 256

__global__ __launch_bounds__(DP_BLOCK) void k_dispatch(DispatchArgs a) {
    __shared__ int wave_cnt[DP_BLOCK / 64];
    __shared__ int s_last;
    __shared__ int s_off[GM_MAX_E + 1];
    const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int total = a.T * a.K;
    int base = 0;
    for (int a0 = 0; a0 < total; a0 += DP_BLOCK * 8) {
        // eight groups of DP_BLOCK assignments per pass, all eight loads in flight
        int v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = a0 + u * DP_BLOCK + tid;
            v[u] = i < total ? a.topk_idx[i] : -1;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = a0 + u * DP_BLOCK + tid;
            const bool match = v[u] == e;
            const unsigned long long bal = __ballot(match);
            const int before = __popcll(bal & ((1ull << lane) - 1ull));
            if (lane == 0) wave_cnt[w] = __popcll(bal);
            __syncthreads();
            int wbase = 0;
            for (int q = 0; q < w; q++) wbase += wave_cnt[q];
            const int tot = wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
            if (match) {
                const int pos = base + wbase + before;  // < T: a token selects an expert at most once
                if (pos < a.T) {
                    __hip_atomic_store(&a.tmp_tok[(size_t)e * a.T + pos], i / a.K, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(&a.tmp_slot[(size_t)e * a.T + pos], i % a.K, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            base += tot;
            __syncthreads();
        }
    }
    if (tid == 0) __hip_atomic_store(&a.counts[e], base < a.T ? base : a.T, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // this thread's write-through stores are done
    __syncthreads();
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(a.E - 1);
    __syncthreads();
    if (!s_last) return;
    // every count in one parallel read, then the prefix in shared memory
    for (int q = tid; q < a.E; q += DP_BLOCK) s_off[q + 1] = __hip_atomic_load(a.counts + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (tid == 0) {
        *a.counter = 0u;
        int off = 0;
        for (int q = 0; q < a.E; q++) {
            const int n = s_off[q + 1];
            s_off[q] = off;
            off += n;
        }
        s_off[a.E] = off;
    }
    __syncthreads();
    for (int q = tid; q <= a.E; q += DP_BLOCK) a.offsets[q] = s_off[q];
    for (int i = tid; i < a.T * a.K; i += DP_BLOCK) a.pair_row[i] = -1;
    __syncthreads();
    // pack: every thread takes up to 8 list positions at a time, all of whose loads are
    // issued together (the position's expert comes from a binary search of the offsets)
    const int listed = s_off[a.E];
    for (int base = 0; base < listed; base += DP_BLOCK * 8) {
        int tk[8], sk[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int pos = base + u * DP_BLOCK + tid;
            tk[u] = sk[u] = 0;
            if (pos < listed) {
                int lo = 0, hi = a.E;  // s_off[lo] <= pos < s_off[hi]
                while (hi - lo > 1) {
                    const int mid = (lo + hi) >> 1;
                    if (s_off[mid] <= pos) lo = mid;
                    else hi = mid;
                }
                tk[u] = __hip_atomic_load(&a.tmp_tok[(size_t)lo * a.T + (pos - s_off[lo])], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                sk[u] = __hip_atomic_load(&a.tmp_slot[(size_t)lo * a.T + (pos - s_off[lo])], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int pos = base + u * DP_BLOCK + tid;
            if (pos < listed) {
                a.tokens[pos] = tk[u];
                a.slots[pos] = sk[u];
                a.pair_row[tk[u] * a.K + sk[u]] = pos;
            }
        }
    }
    if (tid == 0) {
        int nt = 0;
        if (a.routed_on)
            for (int q = 0; q < a.E; q++)
                for (int s = 0; s < s_off[q + 1] - s_off[q]; s += GP_TOK) {
                    const int n = s_off[q + 1] - s_off[q] - s;
                    a.tiles[nt++] = GpTile{q, s_off[q] + s, n < GP_TOK ? n : GP_TOK, 0};
                }
        if (a.shared_on)
            for (int s = 0; s < a.T; s += GP_TOK) a.tiles[nt++] = GpTile{a.E, a.TK + s, a.T - s < GP_TOK ? a.T - s : GP_TOK, 0};
        *a.n_tiles = nt;
    }
}
