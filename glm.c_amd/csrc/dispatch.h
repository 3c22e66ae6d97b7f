// dispatch.h -- per-expert token lists from the per-token top-k (the grouping that the
// reference never materialises: its prefill routes token by token, infer.c:2190-2233).
//
// List e holds every token t with e in topk(t), in ascending t, with the top-k slot it
// came from. One block per expert: it counts every expert's assignments into a shared
// histogram, takes its list's first row and first tile from a prefix over the counts,
// then scans the [T][K] assignments in order and compacts its matches with a ballot
// prefix straight into the packed lists, so the order never depends on atomics and no
// block waits on another.
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
    int *offsets;         // out: [E+1] first list row of each expert, then the rows listed
    int *tokens;          // out: [T*K] token of each list row
    int *slots;           // out: [T*K] top-k slot of each list row
};

#define DP_BLOCK 256

static_assert(GM_MAX_E <= DP_BLOCK, "the offsets' prefix takes one expert per thread");
static_assert(DP_BLOCK == 256, "the list pass gives each of four waves 512 assignments");

__global__ __launch_bounds__(DP_BLOCK) void k_dispatch(DispatchArgs a) {
    __shared__ int hist[GM_MAX_E];
    __shared__ int wave_cnt[DP_BLOCK / 64], wave_tiles[DP_BLOCK / 64];
    __shared__ int s_own[2], s_tot[2];
    const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int total = a.T * a.K;
    if (tid < GM_MAX_E) hist[tid] = 0;
    __syncthreads();
    // every expert's count (eight loads in flight per thread); block 0 marks the
    // assignments that name no expert
    for (int a0 = 0; a0 < total; a0 += DP_BLOCK * 8) {
        int v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = a0 + u * DP_BLOCK + tid;
            v[u] = i < total ? a.topk_idx[i] : 0;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = a0 + u * DP_BLOCK + tid;
            if (i < total) {
                if (v[u] >= 0 && v[u] < a.E) atomicAdd(&hist[v[u]], 1);
                else if (e == 0) a.pair_row[i] = -1;
            }
        }
    }
    __syncthreads();
    // exclusive prefixes of the list lengths (a token selects an expert at most once, so
    // a list holds at most T rows) and of the tiles, one expert per thread
    const int c = tid < a.E ? min(hist[tid], a.T) : 0;
    const int nt = a.routed_on ? (c + GP_TOK - 1) / GP_TOK : 0;
    int ic = c, it = nt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int uc = __shfl_up(ic, o), ut = __shfl_up(it, o);
        if (lane >= o) {
            ic += uc;
            it += ut;
        }
    }
    if (lane == 63) {
        wave_cnt[w] = ic;
        wave_tiles[w] = it;
    }
    __syncthreads();
    for (int q = 0; q < w; q++) {
        ic += wave_cnt[q];
        it += wave_tiles[q];
    }
    if (tid == e) {
        s_own[0] = ic - c;
        s_own[1] = it - nt;
    }
    if (tid == DP_BLOCK - 1) {
        s_tot[0] = ic;
        s_tot[1] = it;
    }
    if (e == 0 && tid < a.E) a.offsets[tid] = ic - c;
    __syncthreads();
    const int own_row = s_own[0], own_cnt = min(hist[e], a.T);
    if (a.routed_on)
        for (int j = tid; j * GP_TOK < own_cnt; j += DP_BLOCK)
            a.tiles[s_own[1] + j] = GpTile{e, own_row + j * GP_TOK, min(GP_TOK, own_cnt - j * GP_TOK), 0};
    if (e == 0) {
        if (a.shared_on)
            for (int j = tid; j * GP_TOK < a.T; j += DP_BLOCK)
                a.tiles[s_tot[1] + j] = GpTile{a.E, a.TK + j * GP_TOK, min(GP_TOK, a.T - j * GP_TOK), 0};
        if (tid == 0) {
            a.offsets[a.E] = s_tot[0];
            *a.n_tiles = s_tot[1] + (a.shared_on ? (a.T + GP_TOK - 1) / GP_TOK : 0);
        }
    }
    // this expert's list, in assignment order: per pass of DP_BLOCK * 8 assignments, wave
    // w takes the contiguous 512 from a0 + 512 w (lane-interleaved, eight loads in
    // flight), keeps its eight match masks, and learns where its matches start from one
    // exchange of the waves' counts
    int base = 0;
    for (int a0 = 0; a0 < total; a0 += DP_BLOCK * 8) {
        const int s0 = a0 + w * 512;
        int v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = s0 + u * 64 + lane;
            v[u] = i < total ? a.topk_idx[i] : -1;
        }
        unsigned long long bal[8];
        int wc = 0;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            bal[u] = __ballot(v[u] == e);
            wc += __popcll(bal[u]);
        }
        if (lane == 0) wave_cnt[w] = wc;
        __syncthreads();
        int pos = base;
        for (int q = 0; q < w; q++) pos += wave_cnt[q];
        base += wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
        const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (v[u] == e) {
                const int i = s0 + u * 64 + lane;
                const int r = pos + __popcll(bal[u] & below);
                if (r < a.T) {
                    a.tokens[own_row + r] = i / a.K;
                    a.slots[own_row + r] = i % a.K;
                    a.pair_row[i] = own_row + r;
                } else {
                    a.pair_row[i] = -1;
                }
            }
            pos += __popcll(bal[u]);
        }
        __syncthreads();  // wave_cnt is rewritten by the next pass
    }
}
