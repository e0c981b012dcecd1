// dispatch.hip -- on-device token -> expert dispatch: histogram, exclusive scan, stable permutation.
//
// The order is ggml mul_mat_id's row mapping, which the reference's wide pass builds on the host
// (byexp at src/server_core_fused.cpp:937; slot tables at :945): for token t ascending and k ascending, pair
// (t, k) = index t*topk + k is appended to its expert's list. perm lists the pairs expert by expert (ascending id),
// each expert's pairs in that order; inv is perm's inverse (the slot of each pair); act lists the used experts
// ascending. One workgroup of 1024 threads: an LDS histogram, a scan, then the pairs in rounds of 1024 where a
// thread's rank among equal experts comes from wave ballots (8 bit-planes of the expert id) plus the counts of the
// waves before it, so the result is the stable counting sort whatever the thread timing. Above 4096 pairs, with a
// scratch buffer, the rounds run as workgroups of their own: k_dispatch_count takes each round's per-expert counts,
// k_dispatch_scan the totals, offsets, used experts and each round's per-expert base (the counts of the rounds before
// it), and k_dispatch_place each round's positions by the same ballots -- the same stable order.
#include "moe_common.h"
#include "moe_kernels.h"

namespace lk {

constexpr int DWAVES = 16;
static_assert(NEXP_MAX % 64 == 0 && NEXP_MAX <= 1024, "the scan's waves and the count's zeroing");

__global__ void __launch_bounds__(1024) k_dispatch(const int * __restrict__ sel, int P, int n_exp, int * __restrict__ counts,
                                                   int * __restrict__ offsets, int * __restrict__ perm, int * __restrict__ inv,
                                                   int * __restrict__ act, int * __restrict__ nact) {
    __shared__ int cnt[NEXP_MAX], base[NEXP_MAX];
    __shared__ int wc[DWAVES][NEXP_MAX];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int e = tid; e < NEXP_MAX; e += 1024) { cnt[e] = 0; }
    __syncthreads();
    for (int i = tid; i < P; i += 1024) {
        const int e = sel[i];
        if (e >= 0 && e < n_exp) { atomicAdd(&cnt[e], 1); }
    }
    __syncthreads();
    if (wave == 0) {   // exclusive scan of the counts and the used-expert list: experts 4 lane .. 4 lane + 3 per lane
        int c[4], s = 0, z = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) { const int e = 4 * lane + j; c[j] = e < n_exp ? cnt[e] : 0; s += c[j]; z += c[j] > 0; }
        int si = s, zi = z;   // inclusive scans over the lanes
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int vs = __shfl_up(si, o), vz = __shfl_up(zi, o);
            if (lane >= o) { si += vs; zi += vz; }
        }
        int acc = si - s, m = zi - z;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 4 * lane + j;
            if (e < n_exp) {
                base[e] = acc; offsets[e] = acc; counts[e] = c[j]; acc += c[j];
                if (c[j] > 0) { act[m++] = e; }
            }
        }
        if (lane == 63) { offsets[n_exp] = si; *nact = zi; }
    }
    __syncthreads();
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int r0 = 0; r0 < P; r0 += 1024) {
        for (int j = tid; j < DWAVES * NEXP_MAX; j += 1024) { (&wc[0][0])[j] = 0; }
        __syncthreads();
        const int i = r0 + tid;
        const int e = i < P ? sel[i] : -1;
        const bool valid = e >= 0 && e < n_exp;
        uint64_t match = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const bool bit = valid && ((e >> b) & 1);
            const uint64_t ones = __ballot(bit);
            match &= bit ? ones : ~ones;
        }
        const int rank = __popcll(match & below);
        if (valid && rank == 0) { wc[wave][e] = __popcll(match); }
        __syncthreads();
        if (valid) {
            int pre = 0;
            for (int w = 0; w < wave; ++w) { pre += wc[w][e]; }
            const int pos = base[e] + pre + rank;
            perm[pos] = i; inv[i] = pos;
        }
        __syncthreads();
        if (tid < n_exp) {
            int s = 0;
            for (int w = 0; w < DWAVES; ++w) { s += wc[w][tid]; }
            base[tid] += s;
        }
        __syncthreads();
    }
}

// round b's per-expert counts: bc[b][e]
__global__ void __launch_bounds__(1024) k_dispatch_count(const int * __restrict__ sel, int P, int n_exp, int * __restrict__ bc) {
    __shared__ int c[NEXP_MAX];
    const int tid = threadIdx.x, i = blockIdx.x * 1024 + tid;
    if (tid < NEXP_MAX) { c[tid] = 0; }
    __syncthreads();
    if (i < P) { const int e = sel[i]; if (e >= 0 && e < n_exp) { atomicAdd(&c[e], 1); } }
    __syncthreads();
    if (tid < n_exp) { bc[blockIdx.x * NEXP_MAX + tid] = c[tid]; }
}
// thread e: expert e's total over the R rounds, the exclusive scans of the totals and of the used flags over the
// experts (wave scans, then the four waves' totals), and round b's base bb[b][e] = offsets[e] + counts of rounds < b
__global__ void __launch_bounds__(NEXP_MAX) k_dispatch_scan(const int * __restrict__ bc, int R, int n_exp, int * __restrict__ counts,
                                                           int * __restrict__ offsets, int * __restrict__ act, int * __restrict__ nact,
                                                           int * __restrict__ bb) {
    __shared__ int ws[NEXP_MAX / 64], wz[NEXP_MAX / 64];
    const int e = threadIdx.x, lane = e & 63, w = e >> 6;
    int tot = 0;
    if (e < n_exp) { for (int b = 0; b < R; ++b) { tot += bc[b * NEXP_MAX + e]; } }
    const int z = tot > 0 ? 1 : 0;
    int si = tot, zi = z;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int vs = __shfl_up(si, o), vz = __shfl_up(zi, o);
        if (lane >= o) { si += vs; zi += vz; }
    }
    if (lane == 63) { ws[w] = si; wz[w] = zi; }
    __syncthreads();
    int ps = 0, pz = 0;
    for (int j = 0; j < w; ++j) { ps += ws[j]; pz += wz[j]; }
    if (e < n_exp) {
        const int excl = ps + si - tot;
        offsets[e] = excl; counts[e] = tot;
        if (z) { act[pz + zi - 1] = e; }
        int acc = excl;
        for (int b = 0; b < R; ++b) { bb[b * NEXP_MAX + e] = acc; acc += bc[b * NEXP_MAX + e]; }
    }
    if (e == NEXP_MAX - 1) { offsets[n_exp] = ps + si; *nact = pz + zi; }
}
// round b's positions: the ballot rank among the wave's equal experts, plus the earlier waves' counts, plus bb[b][e]
__global__ void __launch_bounds__(1024) k_dispatch_place(const int * __restrict__ sel, int P, int n_exp, const int * __restrict__ bb,
                                                         int * __restrict__ perm, int * __restrict__ inv) {
    __shared__ int wc[DWAVES][NEXP_MAX];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int j = tid; j < DWAVES * NEXP_MAX; j += 1024) { (&wc[0][0])[j] = 0; }
    __syncthreads();
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int i = blockIdx.x * 1024 + tid;
    const int e = i < P ? sel[i] : -1;
    const bool valid = e >= 0 && e < n_exp;
    uint64_t match = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const bool bit = valid && ((e >> b) & 1);
        const uint64_t ones = __ballot(bit);
        match &= bit ? ones : ~ones;
    }
    const int rank = __popcll(match & below);
    if (valid && rank == 0) { wc[wave][e] = __popcll(match); }
    __syncthreads();
    if (valid) {
        int pre = 0;
        for (int w = 0; w < wave; ++w) { pre += wc[w][e]; }
        const int pos = bb[blockIdx.x * NEXP_MAX + e] + pre + rank;
        perm[pos] = i; inv[i] = pos;
    }
}

// from DISP_MULTI pairs the rounds run as workgroups (2048 tokens: 40.5 -> 21.9 us); at 4096 pairs and below the
// three launches cost what the one workgroup's rounds do
constexpr int DISP_MULTI = 4097;
size_t dispatch_scratch_ints(int P) { return P >= DISP_MULTI ? (size_t) 2 * ((P + 1023) / 1024) * NEXP_MAX : 0; }

hipError_t launch_dispatch(const int * sel, int P, int n_exp, int * counts, int * offsets, int * perm, int * inv,
                           int * act, int * nact, hipStream_t st, int * scratch) {
    if (n_exp > NEXP_MAX || n_exp <= 0) { return hipErrorInvalidValue; }
    if (P >= DISP_MULTI && scratch) {
        const int R = (P + 1023) / 1024;
        int * bc = scratch, * bb = scratch + (size_t) R * NEXP_MAX;
        k_dispatch_count<<<R, 1024, 0, st>>>(sel, P, n_exp, bc);
        k_dispatch_scan<<<1, NEXP_MAX, 0, st>>>(bc, R, n_exp, counts, offsets, act, nact, bb);
        k_dispatch_place<<<R, 1024, 0, st>>>(sel, P, n_exp, bb, perm, inv);
        return hipGetLastError();
    }
    k_dispatch<<<1, 1024, 0, st>>>(sel, P, n_exp, counts, offsets, perm, inv, act, nact);
    return hipGetLastError();
}

}  // namespace lk
