// moe_device.h -- device-side building blocks of the expert kernels (gfx950, wave64): cross-workgroup exchange, the
// IQ2_XXS x Q8_K block dot product, the in-wave block-order fold and the router's selection. Used by iq2_gemv.hip (one
// kernel per pass) and moe_decode.hip (the single-launch decode block), so both compute bit-identical results.
#pragma once
#include "moe_common.h"

namespace lk {

// ---------------------------------------------------------------- cross-workgroup exchange
// Values one workgroup hands to another inside a launch are written and read with agent-scope relaxed atomics: the XCDs'
// L2 caches are not coherent with each other, and an agent-scope fence would write back / invalidate a whole L2. A
// producer waits for its own stores to complete (vmcnt(0)) before it signals (counter RMW or flag store); a consumer
// issues its loads only after it has seen the signal.
__device__ __forceinline__ void st_agent(float * p, float v) { __hip_atomic_store(gptr(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_agent_u32(uint32_t * p, uint32_t v) { __hip_atomic_store(gptr(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ float ld_agent(const float * p) { return __hip_atomic_load(gptr(const_cast<float *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ uint32_t ld_agent_u32(const uint32_t * p) { return __hip_atomic_load(gptr(const_cast<uint32_t *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ uint64_t ld_agent_u64(const uint64_t * p) { return __hip_atomic_load(gptr(const_cast<uint64_t *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

__device__ __forceinline__ void stores_done() {   // this wave's stores have completed
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// one arrival of the calling wave on a device-scope counter; true for the wave that completes `expected` arrivals,
// which resets the counter for the next launch
__device__ __forceinline__ bool arrive_last(unsigned * cnt, unsigned expected) {
    stores_done();
    unsigned old = 0;
    if (lane_id() == 0) { old = __hip_atomic_fetch_add(gptr(cnt), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
    old = __builtin_amdgcn_readfirstlane(old);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (old + 1 != expected) { return false; }
    if (lane_id() == 0) { __hip_atomic_store(gptr(cnt), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
    return true;
}

// bounded wait of one wave for *flag == want; false after ~2^20 polls (the caller reports the timeout and skips)
__device__ __forceinline__ bool wait_flag(const unsigned * flag, unsigned want) {
    for (int i = 0; i < (1 << 20); ++i) {
        unsigned v = 0;
        if (lane_id() == 0) { v = ld_agent_u32(flag); }
        v = __builtin_amdgcn_readfirstlane(v);
        if (v == want) { __atomic_signal_fence(__ATOMIC_SEQ_CST); return true; }
        __builtin_amdgcn_s_sleep(2);
    }
    return false;
}

// ---------------------------------------------------------------- LDS tables from the prebuilt image
// the table image (layout at TAB_BYTES in moe_common.h) is built once per context in device memory; a workgroup copies it with
// 16-byte loads, all issued before the first LDS write
template <int NT>
__device__ __forceinline__ void tables_copy(uint8_t * lds, const uint4 * img) {
    constexpr int PER = TAB_BYTES / 16 / NT;
    static_assert(PER * NT * 16 == TAB_BYTES, "threads must divide the image");
    uint4 v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) { v[k] = gload16(img + k * NT + threadIdx.x); }
#pragma unroll
    for (int k = 0; k < PER; ++k) { reinterpret_cast<uint4 *>(lds)[k * NT + threadIdx.x] = v[k]; }
}

// The same image rebuilt from 16 bytes per line: each 256-byte line is 16 copies of its first 16 bytes (two copies of a
// codebook entry, or one sign entry), so a workgroup reads 6 KB of the image instead of 96 KB (a launch of 256
// workgroups then moves 1.5 MB through the L2 instead of 24 MB) and writes the copies into LDS. Thread t of nt fills
// the line halves t, t + nt, ..; its k-th write goes to 16-byte slot (k + line) % 8 of its half, so any 16 lanes with
// distinct (line % 8, half) write 16 different bank quads.
__device__ __forceinline__ void tables_fill(const uint8_t * img, LK_LOCAL uint8_t * lds, int t, int nt) {
    for (int p = t; p < 2 * (TAB_BYTES / 256); p += nt) {
        const int line = p >> 1, half = p & 1;
        const u32x4 v = *(const LK_GLOBAL u32x4 *) (img + (size_t) line * 256);
        LK_LOCAL u32x4 * dst = reinterpret_cast<LK_LOCAL u32x4 *>(lds + line * 256 + half * 128);
#pragma unroll
        for (int k = 0; k < 8; ++k) { dst[(k + line) & 7] = v; }
    }
}

// ---------------------------------------------------------------- wave reductions without LDS
// Pure-VALU reductions: DPP inside 16-lane rows (quad_perm xor 1, xor 2, row_half_mirror, row_mirror), then
// row_bcast:15 / row_bcast:31 carry row results upwards so lane 63 ends with the result, read back once. __shfl would
// go through ds_bpermute (the LDS queue the table lookups keep busy), and comparing in scalar registers would bounce
// every step between the vector and scalar units. Keys are 32-bit (a dependent 64-bit compare-select costs ~2x).
enum { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140, DPP_BCAST15 = 0x142, DPP_BCAST31 = 0x143 };
template <int CTRL> __device__ __forceinline__ uint32_t dpp(uint32_t v) { return (uint32_t) __builtin_amdgcn_mov_dpp((int) v, CTRL, 0xF, 0xF, true); }
template <int CTRL> __device__ __forceinline__ float dppf(float v) { return __builtin_bit_cast(float, dpp<CTRL>(__builtin_bit_cast(uint32_t, v))); }
__device__ __forceinline__ uint32_t rdlane(uint32_t v, int l) { return (uint32_t) __builtin_amdgcn_readlane((int) v, l); }

// ---------------------------------------------------------------- router logit contract (shared with the CPU checker)
// K % 1024 == 0: 256 chunks of K/256 consecutive products, each summed in order in fp64 from exact fp32 x fp32 products,
// then a fixed pairwise tree over the chunk sums (entry i of the next level = entries 2i + 2i+1), rounded once to fp32.
// Lane c owns chunks 4c..4c+3 (four independent chains); tree levels 1-2 are lane-local, levels 3-6 pair exactly the
// sibling blocks with DPP inside 16-lane rows (xor 1, xor 2, half mirror, mirror), levels 7-8 combine the four rows.
// fp64 addition is commutative, so which lane of a pair adds which does not change the value.
template <int CTRL> __device__ __forceinline__ double dppd(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = dpp<CTRL>((uint32_t) b), hi = dpp<CTRL>((uint32_t) (b >> 32));
    return __builtin_bit_cast(double, ((uint64_t) hi << 32) | lo);
}
__device__ __forceinline__ double rdlaned(double v, int l) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    return __builtin_bit_cast(double, ((uint64_t) rdlane((uint32_t) (b >> 32), l) << 32) | rdlane((uint32_t) b, l));
}
// tree levels over 64 consecutive chunk sums held one per lane (lane = chunk order): the block's total (uniform)
__device__ __forceinline__ double tree64(double t) {
#pragma clang fp contract(off)
    t = t + dppd<DPP_XOR1>(t);
    t = t + dppd<DPP_XOR2>(t);
    t = t + dppd<DPP_HALF_MIRROR>(t);
    t = t + dppd<DPP_MIRROR>(t);
    return (rdlaned(t, 0) + rdlaned(t, 16)) + (rdlaned(t, 32) + rdlaned(t, 48));
}
// RMSNorm sum of squares (the contract of k_rmsnorm and the decode block's pre-norm): chunk c = 64 q + lane (c = 0..255)
// holds values CL c .. CL c + CL - 1 (CL = 4 L4 = D / 256), summed in order in fp64 from fp32 squares; tree64 over the
// wave's 64 chunks; the four quarters as (q0 + q1) + (q2 + q3).
template <int L4>
__device__ __forceinline__ double sumsq_chunk(const float * row, int c) {
#pragma clang fp contract(off)
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < L4; ++i) {
        const float4 v = gloadf4(row + (size_t) c * 4 * L4 + 4 * i);
        const float q0 = v.x * v.x, q1 = v.y * v.y, q2 = v.z * v.z, q3 = v.w * v.w;
        s += (double) q0; s += (double) q1; s += (double) q2; s += (double) q3;
    }
    return s;
}
// the norm's scale from the four quarter totals
__device__ __forceinline__ float rms_scale(double q0, double q1, double q2, double q3, int D, float eps) {
#pragma clang fp contract(off)
    const double tot = (q0 + q1) + (q2 + q3);
    const float mean = (float) (tot / (double) D);
    return 1.0f / sqrtf(mean + eps);
}
// the lane's four chunk sums -> the wave's total (uniform)
__device__ __forceinline__ double logit_tree(const double (&s)[4]) {
#pragma clang fp contract(off)
    double t = (s[0] + s[1]) + (s[2] + s[3]);
    t = t + dppd<DPP_XOR1>(t);
    t = t + dppd<DPP_XOR2>(t);
    t = t + dppd<DPP_HALF_MIRROR>(t);
    t = t + dppd<DPP_MIRROR>(t);
    return (rdlaned(t, 0) + rdlaned(t, 16)) + (rdlaned(t, 32) + rdlaned(t, 48));
}
// chunk sums of the lane's 4 chunks of w . x (w, x: the row starts); L4 = K / 1024 float4 per chunk
template <int L4>
__device__ __forceinline__ void logit_chunks(const float * w, const float * x, double (&s)[4]) {
#pragma clang fp contract(off)
    const int lane = lane_id();
    const float * wl = w + (size_t) lane * 16 * L4, * xl = x + (size_t) lane * 16 * L4;
#pragma unroll
    for (int j = 0; j < 4; ++j) { s[j] = 0.0; }
#pragma unroll
    for (int i = 0; i < L4; ++i) {
        float4 wv[4], xv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) { wv[j] = gloadf4(wl + j * 4 * L4 + 4 * i); xv[j] = gloadf4(xl + j * 4 * L4 + 4 * i); }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s[j] += (double) xv[j].x * (double) wv[j].x; s[j] += (double) xv[j].y * (double) wv[j].y;
            s[j] += (double) xv[j].z * (double) wv[j].z; s[j] += (double) xv[j].w * (double) wv[j].w;
        }
    }
}
// the same for any K % 1024 == 0 (runtime chunk length)
__device__ __forceinline__ void logit_chunks_any(const float * w, const float * x, int K, double (&s)[4]) {
#pragma clang fp contract(off)
    const int lane = lane_id(), L = K / 256;
    const float * wl = w + (size_t) lane * 4 * L, * xl = x + (size_t) lane * 4 * L;
#pragma unroll
    for (int j = 0; j < 4; ++j) { s[j] = 0.0; }
    for (int i = 0; i < L; i += 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 wv = gloadf4(wl + j * L + i), xv = gloadf4(xl + j * L + i);
            s[j] += (double) xv.x * (double) wv.x; s[j] += (double) xv.y * (double) wv.y;
            s[j] += (double) xv.z * (double) wv.z; s[j] += (double) xv.w * (double) wv.w;
        }
    }
}

// wave-wide maximum of unsigned 32-bit values, returned to every lane (uniform). Every step reads its partner through
// DPP with bound_ctrl (lanes without a partner read 0, the identity of max), so each step is one v_max_u32_dpp; after
// row_bcast:15 / row_bcast:31 lane 63 holds the maximum of all 64 lanes.
__device__ __forceinline__ uint32_t umax32(uint32_t a, uint32_t b) { return a > b ? a : b; }
template <int CTRL> __device__ __forceinline__ uint32_t max32_step(uint32_t v) { return umax32(v, dpp<CTRL>(v)); }
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max32_step<DPP_XOR1>(v); v = max32_step<DPP_XOR2>(v);
    v = max32_step<DPP_HALF_MIRROR>(v); v = max32_step<DPP_MIRROR>(v);
    v = max32_step<DPP_BCAST15>(v); v = max32_step<DPP_BCAST31>(v);
    return rdlane(v, 63);
}
// inclusive prefix sum over the wave's lanes (lane l gets v_0 + .. + v_l): shifts inside 16-lane rows, then each row adds
// the totals of the rows below it (row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2 and 3)
template <int CTRL, int ROWS> __device__ __forceinline__ uint32_t scan_step(uint32_t v) {
    return v + (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, CTRL, ROWS, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t v) {
    v = scan_step<0x111, 0xF>(v); v = scan_step<0x112, 0xF>(v); v = scan_step<0x114, 0xF>(v); v = scan_step<0x118, 0xF>(v);
    v = scan_step<DPP_BCAST15, 0xA>(v); v = scan_step<DPP_BCAST31, 0xC>(v);
    return v;
}
// lowest lane whose flag is set (uniform; 64 if none)
__device__ __forceinline__ int first_lane(bool f) { const uint64_t b = __ballot(f); return b ? __builtin_ctzll(b) : 64; }

// fp32 bits -> unsigned key with the same order (no -0 / NaN among the values compared here)
__device__ __forceinline__ uint32_t ord_key(float f) { const uint32_t b = __builtin_bit_cast(uint32_t, f); return (b & 0x80000000u) ? ~b : (b | 0x80000000u); }

// ---------------------------------------------------------------- Q8_K of one 256-value block by one wave
// quantize_row_q8_K_ref: lane l holds values 4l..4l+3; amax with its first occurrence's signed value, iscale = -127/max,
// q = min(127, round-half-even(iscale * x)), d = 1/iscale; an all-zero block gives d = 0. Returns the lane's 4 packed q.
__device__ __forceinline__ uint32_t q8k_lane(const float (&xs)[4], float & d) {
#pragma clang fp contract(off)
    const int lane = lane_id();
    float ba = -1.f, bv = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) { const float ax = fabsf(xs[i]); if (ax > ba) { ba = ax; bv = xs[i]; } }
    // the largest |x| (non-negative floats order as their bits); ties to the lower index = the lowest lane holding the
    // maximum, whose own best is its lowest such index
    const uint32_t mk = wave_max_u32(__builtin_bit_cast(uint32_t, ba));
    const int wl = first_lane(__builtin_bit_cast(uint32_t, ba) == mk);
    ba = __builtin_bit_cast(float, mk);
    bv = __builtin_bit_cast(float, rdlane(__builtin_bit_cast(uint32_t, bv), wl));
    uint32_t packed = 0; d = 0.f;
    if (ba > 0.f) {
        const float iscale = -127.f / bv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = iscale * xs[i];
            int iv = (int) rintf(p); iv = iv < 127 ? iv : 127;
            packed |= ((uint32_t) (iv & 0xff)) << (8 * i);
        }
        d = 1.f / iscale;
    }
    return packed;
}

// Q8_K of four blocks at once, one per 16-lane row: lane 16 m + i holds values 16 i .. 16 i + 15 of row m's block. The
// operations and tie rules are q8k_lane's (largest |x|, its first occurrence's signed value; q = min(127,
// round-half-even(iscale * x)), d = 1 / iscale), with the reductions inside the row: max of |x| by DPP, then the lowest
// lane holding it (DPP min), whose value ds_bpermute fetches. packed[w] = values 16 i + 4 w .. + 3; d = the row's scale.
__device__ __forceinline__ void q8k_row16(const float (&xs)[16], uint32_t (&packed)[4], float & d) {
#pragma clang fp contract(off)
    const int lane = lane_id(), i = lane & 15;
    float ba = -1.f, bv = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) { const float ax = fabsf(xs[k]); if (ax > ba) { ba = ax; bv = xs[k]; } }
    uint32_t mk = __builtin_bit_cast(uint32_t, ba);
    mk = umax32(mk, dpp<DPP_XOR1>(mk)); mk = umax32(mk, dpp<DPP_XOR2>(mk));
    mk = umax32(mk, dpp<DPP_HALF_MIRROR>(mk)); mk = umax32(mk, dpp<DPP_MIRROR>(mk));
    uint32_t c = __builtin_bit_cast(uint32_t, ba) == mk ? (uint32_t) i : 16u;
    c = min(c, dpp<DPP_XOR1>(c)); c = min(c, dpp<DPP_XOR2>(c));
    c = min(c, dpp<DPP_HALF_MIRROR>(c)); c = min(c, dpp<DPP_MIRROR>(c));
    const float vmax = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((int) (((lane & 48) | c) * 4), __builtin_bit_cast(int, bv)));
    const bool nz = __builtin_bit_cast(float, mk) > 0.f;
    const float iscale = -127.f / (nz ? vmax : 1.f);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t pk = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float p = iscale * xs[4 * w + b];
            int iv = (int) rintf(p); iv = iv < 127 ? iv : 127;
            pk |= ((uint32_t) (iv & 0xff)) << (8 * b);
        }
        packed[w] = nz ? pk : 0u;
    }
    d = nz ? 1.f / iscale : 0.f;
}

// ---------------------------------------------------------------- staged activations
// BPQ blocks per K quarter (4 quarters); lane 4 r + q of a task owns row r and blocks j = 4 jj + q, so the 4 lanes of a
// quad hold 4 consecutive blocks of one row at every step. One token's staged activations: per block 256 int8 (+16 B of
// padding, so the quarters' reads of one instruction fall in different banks) re-ordered so that group l of all 8
// sub-blocks is contiguous (byte l * 64 + ib * 8 + k = x[ib * 32 + l * 8 + k]), then the NB fp32 block scales.
// PAD: bytes after each staged block (the per-pass kernels' lanes read 4 different blocks at once: 16 bytes of padding
// put them in different banks; the decode block's lanes read one block at a time and stage without padding)
template <int BPQ_, int PAD = 16> struct Geo {
    static constexpr int QS = 4, BPQ = BPQ_, RPW = 16, NB = QS * BPQ, K = NB * QK;
    static constexpr int XBLK = QK + PAD, XROW = NB * XBLK + NB * 4;
};
// staged byte offset inside a block of the 4 values 4 lane .. 4 lane + 3 (sub-block lane / 8, group (lane % 8) / 2)
__device__ __forceinline__ int staged_word(int lane) { return ((lane & 7) >> 1) * 64 + (lane >> 3) * 8 + (lane & 1) * 4; }

// one token row of Q8_K values (K int8 + NB scales in global memory) into the staged layout, by one wave
template <class G>
__device__ __forceinline__ void stage_row(uint8_t * dst, const int8_t * src, const float * dsrc) {
    const int lane = lane_id();
    constexpr int IT = G::K / 8 / 64;
    uint2 v[IT];
#pragma unroll
    for (int it = 0; it < IT; ++it) { v[it] = gload8(src + (size_t) (it * 64 + lane) * 8); }
    const float dv = lane < G::NB ? gptr(dsrc)[lane] : 0.f;
#pragma unroll
    for (int it = 0; it < IT; ++it) {   // 8-byte piece i = (block j, sub-block ib, group l)
        const int i = it * 64 + lane, j = i >> 5, w = i & 31;
        *reinterpret_cast<uint2 *>(dst + j * G::XBLK + (w & 3) * 64 + (w >> 2) * 8) = v[it];
    }
    if (lane < G::NB) { reinterpret_cast<float *>(dst + G::NB * G::XBLK)[lane] = dv; }
}
// the same from values another workgroup wrote in this launch (agent-scope loads)
template <class G>
__device__ __forceinline__ void stage_row_agent(uint8_t * dst, const int8_t * src, const float * dsrc) {
    const int lane = lane_id();
    constexpr int IT = G::K / 8 / 64;
    uint64_t v[IT];
#pragma unroll
    for (int it = 0; it < IT; ++it) { v[it] = ld_agent_u64(reinterpret_cast<const uint64_t *>(src) + it * 64 + lane); }
    const float dv = lane < G::NB ? ld_agent(dsrc + lane) : 0.f;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int i = it * 64 + lane, j = i >> 5, w = i & 31;
        *reinterpret_cast<uint64_t *>(dst + j * G::XBLK + (w & 3) * 64 + (w >> 2) * 8) = v[it];
    }
    if (lane < G::NB) { reinterpret_cast<float *>(dst + G::NB * G::XBLK)[lane] = dv; }
}
__device__ __forceinline__ void lds_visible() {   // this wave's LDS writes are done before any of its lanes reads them
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
}

// ---------------------------------------------------------------- one block: integer sums of T tokens
template <int L, int T>
__device__ __forceinline__ void group_step(const uint4 (&w)[4], uint32_t tr, const uint8_t * const (&xb)[T], int (&acc)[T][8]) {
    const uint32_t trs = tab_sign_word(tr);
    uint2 g[8]; uint4 m[8];   // all 16 table reads of the step are issued before the first is used
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {
        const uint4 c = w[ib >> 1];
        g[ib] = tab_grid<L>((ib & 1) ? c.z : c.x, tr);
        m[ib] = tab_sign<L>(((ib & 1) ? c.w : c.y) & SIGN_BITS, trs);
    }
    int4 xv[T][4];
#pragma unroll
    for (int u = 0; u < T; ++u) {
#pragma unroll
        for (int k = 0; k < 4; ++k) { xv[u][k] = *reinterpret_cast<const int4 *>(xb[u] + L * 64 + k * 16); }
    }
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {
        uint32_t lo, hi; iq2_apply(g[ib], m[ib], lo, hi);
#pragma unroll
        for (int u = 0; u < T; ++u) {
            const int4 x = xv[u][ib >> 1];
            acc[u][ib] = __builtin_amdgcn_sdot4((int) lo, (ib & 1) ? x.z : x.x, acc[u][ib], false);
            acc[u][ib] = __builtin_amdgcn_sdot4((int) hi, (ib & 1) ? x.w : x.y, acc[u][ib], false);
        }
    }
}

// exact integer block sums sum_ib (2 nibble_ib + 1) * sumi_ib of one IQ2_XXS block (tiled chunks w) against T tokens
template <int T>
__device__ __forceinline__ void block_bsum(const uint4 (&w)[4], uint32_t tr, const uint8_t * const (&xb)[T], int (&bsum)[T]) {
    int acc[T][8];
#pragma unroll
    for (int u = 0; u < T; ++u) {
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) { acc[u][ib] = 0; }
    }
    group_step<0, T>(w, tr, xb, acc);
    group_step<1, T>(w, tr, xb, acc);
    group_step<2, T>(w, tr, xb, acc);
    group_step<3, T>(w, tr, xb, acc);
#pragma unroll
    for (int u = 0; u < T; ++u) {
        int s = 0;
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) {   // |acc| <= 32 * 43 * 127 < 2^23: the 24-bit multiply is exact
            const uint4 c = w[ib >> 1];
            s += __mul24(acc[u][ib], iq2_scale((ib & 1) ? c.w : c.y));
        }
        bsum[u] = s;
    }
}

template <int Q> __device__ __forceinline__ float quad_bcast(float v) {   // lane Q of every quad, to the whole quad
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), Q * 0x55, 0xF, 0xF, true));
}
// the 4 lanes of a quad hold consecutive blocks 4 jj .. 4 jj + 3 of one row: add their terms in block order
__device__ __forceinline__ float fold_quad(float acc, float t) {
#pragma clang fp contract(off)
    acc = acc + quad_bcast<0>(t);
    acc = acc + quad_bcast<1>(t);
    acc = acc + quad_bcast<2>(t);
    return acc + quad_bcast<3>(t);
}

// ---------------------------------------------------------------- the same product with the activations in registers
// Lane layout 16 q + r (q = block quarter, r = row): the 16 lanes of a DPP row share one activation block, so each lane
// holds 4 of its 64 dwords (dwords 4r .. 4r + 3 of the staged block) and every dot product reads its dword by
// row_newbcast from the lane that holds it -- one LDS read per block instead of 16. Staged dword 16 L + 2 ib + hi
// (group L, sub-block ib, weights 0..3 / 4..7) lives in lane 4 L + ib / 2, register 2 (ib & 1) + hi.
template <int CTRL> __device__ __forceinline__ int dppi(int v) { return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false); }
// acc += dot4(x of lane SRC of this lane's DPP row, w): v_dot4c_i32_i8 with the broadcast as its DPP source modifier,
// one instruction where v_mov_b32_dpp + v_dot4c took two (the compiler does not fold row_newbcast into the dot; the
// block product is VALU-bound at 16 waves per CU, and this removes 64 of its ~300 instructions per 256 weights).
// The DPP source must not be written by a VALU instruction in the two wait states before: the compiler does not see
// the DPP inside the asm, so the callers pass LDS-loaded words (xq, from ds_read), and tests/test_isa.py checks the
// built library's disassembly for such a write.
template <int SRC> __device__ __forceinline__ int dot4_bcast(int acc, uint32_t x, uint32_t w) {
    asm("v_dot4c_i32_i8_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(x), "v"(w), "i"(SRC));
    return acc;
}
template <int L, int IB, int IBE = 8>
__device__ __forceinline__ void dot_ib_dpp(const uint2 (&g)[8], const uint4 (&m)[8], const uint32_t (&xq)[4], int (&acc)[8]) {
    if constexpr (IB < IBE) {
        uint32_t lo, hi; iq2_apply(g[IB], m[IB], lo, hi);
        constexpr int SRC = 4 * L + IB / 2;
        acc[IB] = dot4_bcast<SRC>(acc[IB], xq[2 * (IB & 1)], lo);
        acc[IB] = dot4_bcast<SRC>(acc[IB], xq[2 * (IB & 1) + 1], hi);
        dot_ib_dpp<L, IB + 1, IBE>(g, m, xq, acc);
    }
}
// the group's 16 table reads in batches of IBB sub-blocks (8: all issued before the first is used; 4: half the registers)
#ifndef LK_IBB
#define LK_IBB 8
#endif
template <int L, int IB0 = 0>
__device__ __forceinline__ void group_step_dpp(const uint4 (&w)[4], uint32_t tr, const uint32_t (&xq)[4], int (&acc)[8]) {
    if constexpr (IB0 < 8) {
        const uint32_t trs = tab_sign_word(tr);
        uint2 g[8]; uint4 m[8];
#pragma unroll
        for (int ib = IB0; ib < IB0 + LK_IBB; ++ib) {
            const uint4 c = w[ib >> 1];
            g[ib] = tab_grid<L>((ib & 1) ? c.z : c.x, tr);
            m[ib] = tab_sign<L>(((ib & 1) ? c.w : c.y) & SIGN_BITS, trs);
        }
        dot_ib_dpp<L, IB0, IB0 + LK_IBB>(g, m, xq, acc);
        group_step_dpp<L, IB0 + LK_IBB>(w, tr, xq, acc);
    }
}
// block_bsum for one token whose staged block is xb (this lane reads its 16 bytes at xb + 16 r)
__device__ __forceinline__ int block_bsum_dpp(const uint4 (&w)[4], uint32_t tr, const uint8_t * xb, int r) {
    const u32x4 xv = *(const LK_LOCAL u32x4 *) (size_t) lds_addr(xb + 16 * r);
    const uint32_t xq[4] = { xv.x, xv.y, xv.z, xv.w };
    int acc[8];
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) { acc[ib] = 0; }
    group_step_dpp<0>(w, tr, xq, acc);
    group_step_dpp<1>(w, tr, xq, acc);
    group_step_dpp<2>(w, tr, xq, acc);
    group_step_dpp<3>(w, tr, xq, acc);
    int s = 0;
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {   // |acc| <= 32 * 43 * 127 < 2^23: the 24-bit multiply is exact
        const uint4 c = w[ib >> 1];
        s += __mul24(acc[ib], iq2_scale((ib & 1) ? c.w : c.y));
    }
    return s;
}
// lanes 16 q + r hold the terms of blocks 4 jj + q of row r: lanes 0..15 add the four in block order (lanes 16..63 are
// left with partial values). v_permlane16_swap v, z exchanges v's rows 1 and 3 with z's rows 0 and 2, so z then holds
// v's lanes 16..31 in lanes 0..15; v_permlane32_swap v, z exchanges v's lanes 32..63 with z's lanes 0..31. Written as
// inline assembly so that which register receives which half is fixed (s_nop 1: the wait states a VALU result needs
// before a permlane reads it).
__device__ __forceinline__ uint32_t lanes_16_31(uint32_t v) {
    uint32_t z = 0;
    __asm__ volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(v), "+v"(z));
    return z;
}
__device__ __forceinline__ uint32_t lanes_32_63(uint32_t v) {
    uint32_t z = 0;
    __asm__ volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(v), "+v"(z));
    return z;
}
__device__ __forceinline__ float fold_rows(float acc, float t) {
#pragma clang fp contract(off)
    const uint32_t b = __builtin_bit_cast(uint32_t, t);
    const uint32_t hi = lanes_32_63(b);   // lanes 0..15: q = 2, lanes 16..31: q = 3
    acc = acc + t;
    acc = acc + __builtin_bit_cast(float, lanes_16_31(b));
    acc = acc + __builtin_bit_cast(float, hi);
    return acc + __builtin_bit_cast(float, lanes_16_31(hi));
}

// ---------------------------------------------------------------- streaming RPL x 16 rows of one matrix
// Steps s = 0 .. RPL * BPQ - 1: row set s / BPQ (16 rows each, 256 B apart in a tiled chunk), block step jj = s % BPQ.
// qb / db: uniform qs / d bases of the task's first row set at jj = 0; lq / ld: the lane's part of its addresses.
template <int BPQ, int RPL, int PD>
struct RowStream {
    static constexpr int STEPS = RPL * BPQ, NR = PD + 1;
    uint4 pf[NR][4]; uint16_t pd[NR];
    __device__ __forceinline__ void issue(const uint8_t * qb, const uint8_t * db, uint32_t lq, uint32_t ld, int s, int slot) {
        const int rs = s / BPQ, jj = s % BPQ;
        const uint8_t * q = qb + (size_t) rs * 256 + (size_t) jj * (4 * 4096);
#pragma unroll
        for (int c = 0; c < 4; ++c) { pf[slot][c] = load_nt(q + lq + c * 1024); }
        pd[slot] = *gptr(reinterpret_cast<const uint16_t *>(db + (size_t) rs * 32 + (size_t) jj * (4 * 128) + ld));
    }
    // steps [K0, K1) of the first PD (run issues the rest); prologue = all of them
    template <int K0 = 0, int K1 = PD>
    __device__ __forceinline__ void prologue(const uint8_t * qb, const uint8_t * db, uint32_t lq, uint32_t ld) {
#pragma unroll
        for (int k = K0; k < K1; ++k) { if (k < STEPS) { issue(qb, db, lq, ld, k, k); } }
    }
    // row totals (before the final * 0.125) of the lane's RPL rows for T staged tokens xr[u]
    template <int T, class G>
    __device__ __forceinline__ void run(const uint8_t * qb, const uint8_t * db, uint32_t lq, uint32_t ld, uint32_t tr,
                                        const uint8_t * const (&xr)[T], int q, float (&acc)[RPL][T]) {
#pragma clang fp contract(off)
#pragma unroll
        for (int rs = 0; rs < RPL; ++rs) {
#pragma unroll
            for (int u = 0; u < T; ++u) { acc[rs][u] = 0.f; }
        }
#pragma unroll 1
        for (int s0 = 0; s0 < STEPS; s0 += NR) {
#pragma unroll
            for (int k = 0; k < NR; ++k) {
                const int s = s0 + k;
                if (s < STEPS) {
                    if (s + PD < STEPS) { issue(qb, db, lq, ld, s + PD, (k + PD) % NR); }
                    const int j = (s % BPQ) * 4 + q;
                    const uint8_t * xb[T];
#pragma unroll
                    for (int u = 0; u < T; ++u) { xb[u] = xr[u] + j * G::XBLK; }
                    int bsum[T];
                    block_bsum<T>(pf[k], tr, xb, bsum);
                    const float dw = h2f(pd[k]);
                    const int rs = s / BPQ;
#pragma unroll
                    for (int u = 0; u < T; ++u) {
                        const float dx = reinterpret_cast<const float *>(xr[u] + G::NB * G::XBLK)[j];
                        const float t = (dw * dx) * (float) bsum[u];
                        // rs is uniform: select the accumulator without dynamic register indexing
#pragma unroll
                        for (int r2 = 0; r2 < RPL; ++r2) { if (r2 == rs) { acc[r2][u] = fold_quad(acc[r2][u], t); } }
                    }
                }
            }
        }
    }
    // the same for one token with the activations in registers (lane layout 16 q + r; totals valid in lanes 0..15)
    template <class G>
    __device__ __forceinline__ void run_dpp(const uint8_t * qb, const uint8_t * db, uint32_t lq, uint32_t ld, uint32_t tr,
                                            const uint8_t * xr, int q, int r, float (&acc)[RPL]) {
#pragma clang fp contract(off)
#pragma unroll
        for (int rs = 0; rs < RPL; ++rs) { acc[rs] = 0.f; }
#pragma unroll 1
        for (int s0 = 0; s0 < STEPS; s0 += NR) {
#pragma unroll
            for (int k = 0; k < NR; ++k) {
                const int s = s0 + k;
                if (s < STEPS) {
                    if (s + PD < STEPS) { issue(qb, db, lq, ld, s + PD, (k + PD) % NR); }
                    const int j = (s % BPQ) * 4 + q;
                    const int bsum = block_bsum_dpp(pf[k], tr, xr + j * G::XBLK, r);
                    const float dx = reinterpret_cast<const float *>(xr + G::NB * G::XBLK)[j];
                    const float t = (h2f(pd[k]) * dx) * (float) bsum;
                    const int rs = s / BPQ;
#pragma unroll
                    for (int r2 = 0; r2 < RPL; ++r2) { if (r2 == rs) { acc[r2] = fold_rows(acc[r2], t); } }
                }
            }
        }
    }
};

// ---------------------------------------------------------------- router selection of one token by one wave

// Grouped sigmoid top-k (the rule of router.hip): p = sigmoid(logit), c = p + bias; group score = top1 + top2 of c in
// the group; groups ranked by score (ties to the lower group) keep topk_group; topk rounds of argmax over eligible
// experts (ties to the lower index); w_r = p_r / max(sum_r p_r, 2^-14) * scale with the sum in pick order.
// keep < topk then keeps the keep largest weights (the engine's narrow dispatch, src/server_core_fused.cpp:793-811):
// ordered by weight descending, equal weights in pick order, and, with renorm > 0, every kept weight multiplied by
// f = renorm / sw when the kept sum sw (in kept order, fp32) exceeds 1e-6. sel_out / w_out receive keep entries.
// lg[j] = logit of expert 4 lane + j. scr: per-wave LDS scratch of n_exp + 2 * n_group floats (general group sizes only).
template <int CTRL> __device__ __forceinline__ void top2_step(float & v1, float & v2) {
    const float o1 = dppf<CTRL>(v1), o2 = dppf<CTRL>(v2);
    const float n2 = v1 >= o1 ? fmaxf(v2, o1) : fmaxf(v1, o2);
    v1 = fmaxf(v1, o1); v2 = n2;
}
// the lane's 4 bias values (experts 4 lane + j), loaded ahead of the logits
__device__ __forceinline__ void load_bias(const float * bias, int n_exp, float (&b)[4]) {
    const int lane = lane_id();
#pragma unroll
    for (int j = 0; j < 4; ++j) { b[j] = 4 * lane + j < n_exp ? gptr(bias)[4 * lane + j] : 0.f; }
}
// the rule from the lane's 4 probabilities p[j] = sigmoid(logit) of experts 4 lane + j
// SCRATCH = false: the caller guarantees the DPP group path (decode_rule_ok) and passes no scratch
template <bool SCRATCH = true>
__device__ __forceinline__ void select_token_p(const float (&p)[4], const float (&bias)[4], int n_exp, int n_group, int topk_group, int topk,
                                               float scale, float * scr, int * sel_out, float * w_out, int keep, float renorm) {
#pragma clang fp contract(off)
    const int lane = lane_id(), per = n_exp / n_group;
    float c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) { c[j] = 4 * lane + j < n_exp ? p[j] + bias[j] : 0.f; }
    bool ok[4];
    const int lpg = per / 4;   // lanes per group
    if (per % 4 == 0 && (lpg & (lpg - 1)) == 0 && lpg <= 16) {
        // top1 / top2 of the group: the lane's 4, then across the group's lanes (DPP inside a 16-lane row)
        float v1 = -INFINITY, v2 = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (4 * lane + j < n_exp) { const float v = c[j]; if (v > v1) { v2 = v1; v1 = v; } else if (v > v2) { v2 = v; } }
        }
        if (lpg >= 2) { top2_step<DPP_XOR1>(v1, v2); }
        if (lpg >= 4) { top2_step<DPP_XOR2>(v1, v2); }
        if (lpg >= 8) { top2_step<DPP_HALF_MIRROR>(v1, v2); }
        if (lpg >= 16) { top2_step<DPP_MIRROR>(v1, v2); }
        const float mine = v1 + v2;   // this lane's group score
        const int gme = lane / lpg;
        int rank = 0;
        for (int h = 0; h < n_group; ++h) {   // a group stays eligible if fewer than topk_group groups beat it
            const float o = __builtin_bit_cast(float, rdlane(__builtin_bit_cast(uint32_t, mine), h * lpg));
            rank += (o > mine || (o == mine && h < gme)) ? 1 : 0;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) { ok[j] = 4 * lane + j < n_exp && rank < topk_group; }
    } else if constexpr (!SCRATCH) {
#pragma unroll
        for (int j = 0; j < 4; ++j) { ok[j] = false; }   // not reached (the caller checked the rule)
    } else {
        float * cs = scr; float * gsc = scr + n_exp; int * allow = reinterpret_cast<int *>(scr + n_exp + n_group);
#pragma unroll
        for (int j = 0; j < 4; ++j) { if (4 * lane + j < n_exp) { cs[4 * lane + j] = c[j]; } }
        lds_visible();
        if (lane < n_group) {   // top1 + top2 of the group's biased scores
            float v1 = 0.f, v2 = 0.f; int i1 = -1, i2 = -1;
            for (int e = lane * per; e < (lane + 1) * per; ++e) {
                const float v = cs[e];
                if (i1 < 0 || v > v1) { v2 = v1; i2 = i1; v1 = v; i1 = e; }
                else if (i2 < 0 || v > v2) { v2 = v; i2 = e; }
            }
            gsc[lane] = v1 + v2;
        }
        lds_visible();
        if (lane < n_group) {
            int rank = 0; const float mine = gsc[lane];
            for (int h = 0; h < n_group; ++h) { const float o = gsc[h]; rank += (o > mine || (o == mine && h < lane)) ? 1 : 0; }
            allow[lane] = rank < topk_group;
        }
        lds_visible();
#pragma unroll
        for (int j = 0; j < 4; ++j) { const int e = 4 * lane + j; ok[j] = e < n_exp && allow[e / per]; }
    }
    // topk rounds of argmax over the eligible, untaken experts: the largest ordered key of c; ties to the lower index.
    // Each lane first sorts its 4 (key, p, j) by key, descending and stably (adjacent exchanges on a strictly larger
    // key: among equal keys the lower j stays first), so a round only reads the lanes' heads: the winner is the lowest
    // lane whose head holds the maximum, and that lane drops its head.
    uint32_t kk[4]; float pp[4]; int jj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) { kk[j] = ok[j] ? ord_key(c[j]) : 0u; pp[j] = p[j]; jj[j] = j; }
    auto cex = [&](int x, int y) {
        const bool sw = kk[y] > kk[x];
        const uint32_t k0 = kk[x]; const float p0 = pp[x]; const int j0 = jj[x];
        kk[x] = sw ? kk[y] : kk[x]; pp[x] = sw ? pp[y] : pp[x]; jj[x] = sw ? jj[y] : jj[x];
        kk[y] = sw ? k0 : kk[y]; pp[y] = sw ? p0 : pp[y]; jj[y] = sw ? j0 : jj[y];
    };
    cex(0, 1); cex(1, 2); cex(2, 3); cex(0, 1); cex(1, 2); cex(0, 1);
    float sum = 0.f, p_mine = 0.f; int sel_mine = -1;   // lane r keeps round r's pick
    for (int r = 0; r < topk; ++r) {
        const uint32_t m = wave_max_u32(kk[0]);
        int bi = -1; float bp = 0.f;
        if (m) {
            const int wl = first_lane(kk[0] == m);
            bi = 4 * wl + (int) rdlane((uint32_t) jj[0], wl);
            bp = __builtin_bit_cast(float, rdlane(__builtin_bit_cast(uint32_t, pp[0]), wl));
            if (lane == wl) {
                kk[0] = kk[1]; kk[1] = kk[2]; kk[2] = kk[3]; kk[3] = 0u;
                pp[0] = pp[1]; pp[1] = pp[2]; pp[2] = pp[3];
                jj[0] = jj[1]; jj[1] = jj[2]; jj[2] = jj[3];
            }
        }
        sum = sum + bp;
        if (lane == r) { sel_mine = bi; p_mine = bp; }
    }
    sum = sum > 6.103515625e-5f ? sum : 6.103515625e-5f;
    const float w_mine = p_mine / sum * scale;
    if (keep >= topk) {
        if (lane < topk) { sel_out[lane] = sel_mine; w_out[lane] = w_mine; }
        return;
    }
    // rank of lane r's weight among the topk picks: heavier picks, then equal ones picked earlier
    int rank = 0;
    for (int j = 0; j < topk; ++j) {
        const float o = __builtin_bit_cast(float, rdlane(__builtin_bit_cast(uint32_t, w_mine), j));
        rank += (o > w_mine || (o == w_mine && j < lane)) ? 1 : 0;
    }
    const bool kept = lane < topk && rank < keep;
    float f = 1.f; bool rescale = false;
    if (renorm > 0.f) {
        float sw = 0.0f;
        for (int q = 0; q < keep; ++q) {   // the kept weights in kept order
            const int l = first_lane(lane < topk && rank == q);
            sw = sw + __builtin_bit_cast(float, rdlane(__builtin_bit_cast(uint32_t, w_mine), l));
        }
        if (sw > 1e-6f) { f = renorm / sw; rescale = true; }
    }
    if (kept) { sel_out[rank] = sel_mine; w_out[rank] = rescale ? w_mine * f : w_mine; }
}
// DeepSeek's rule (256 experts, 8 groups of 32, 4 groups kept, top 8 kept whole) on one wave, with the same picks in
// the same order and the same weights as select_token_p, in far fewer dependent steps. The group stage is
// select_token_p's. Then, instead of 8 rounds of a wave-wide argmax: L = the smallest second-best c of the kept groups.
// The kept groups' best and second-best are 8 distinct eligible experts with c >= L, so the 8th largest eligible c is
// at least L and every pick is among the candidates {eligible e : c_e >= L}. The candidates (usually 8-14) are
// compacted into scr and each is ranked against the others by (c descending, index ascending) -- the rounds' order,
// ties to the lower index -- which gives pick r = the candidate of rank r. The weights follow as in select_token_p:
// the sum in pick order, clamped, p / sum * scale. Falls back (returns false, outputs untouched) if some c is NaN (c
// is never -0: p > 0 or p = +0) or more than 32 candidates remain. scr: 112 words of LDS.
__device__ __forceinline__ bool select_ds8(const float (&p)[4], const float (&bias)[4], float scale, LK_LOCAL uint32_t * scr,
                                           int * sel_out, float * w_out) {
#pragma clang fp contract(off)
    const int lane = lane_id();
    float c[4];
    bool nan = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) { c[j] = p[j] + bias[j]; nan = nan || c[j] != c[j]; }
    if (__ballot(nan)) { return false; }
    float v1 = -INFINITY, v2 = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) { const float v = c[j]; if (v > v1) { v2 = v1; v1 = v; } else if (v > v2) { v2 = v; } }
    top2_step<DPP_XOR1>(v1, v2); top2_step<DPP_XOR2>(v1, v2); top2_step<DPP_HALF_MIRROR>(v1, v2);   // 8 lanes per group
    const float mine = v1 + v2;
    const int gme = lane >> 3;
    int rank = 0;
#pragma unroll
    for (int h = 0; h < 8; ++h) {
        const float o = __builtin_bit_cast(float, rdlane(__builtin_bit_cast(uint32_t, mine), h * 8));
        rank += (o > mine || (o == mine && h < gme)) ? 1 : 0;
    }
    const bool elig = rank < 4;
    // L as an ordered key: the minimum over the kept groups of ord_key(v2)
    const uint32_t lk = ~wave_max_u32(elig ? ~ord_key(v2) : 0u);
    uint32_t kk[4]; int cand = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) { kk[j] = ord_key(c[j]); cand |= (elig && kk[j] >= lk) ? 1 << j : 0; }
    const uint32_t cnt = (uint32_t) __builtin_popcount(cand), incl = wave_scan_u32(cnt);
    const int ncand = (int) rdlane(incl, 63);
    if (ncand < 8 || ncand > 32) { return false; }
    // compact: candidate i at scr[i] (key), scr[32 + i] (index), scr[64 + i] (p)
    int at = (int) (incl - cnt);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (cand & (1 << j)) { scr[at] = kk[j]; scr[32 + at] = (uint32_t) (4 * lane + j); scr[64 + at] = __builtin_bit_cast(uint32_t, p[j]); ++at; }
    }
    lds_visible();
    const bool mine_c = lane < ncand;
    const uint32_t ki = mine_c ? scr[lane] : 0u, ii = mine_c ? scr[32 + lane] : 0u;
    int rk = 0;
    for (int t0 = 0; t0 < ncand; t0 += 4) {
        const u32x4 kt = *reinterpret_cast<const LK_LOCAL u32x4 *>(scr + t0), it = *reinterpret_cast<const LK_LOCAL u32x4 *>(scr + 32 + t0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            rk += (t0 + q < ncand && (kt[q] > ki || (kt[q] == ki && it[q] < ii))) ? 1 : 0;
        }
    }
    lds_visible();   // every lane has read the candidates before the picks overwrite the index words
    if (mine_c && rk < MAXK) { scr[96 + rk] = ii; scr[104 + rk] = scr[64 + lane]; }
    lds_visible();
    const u32x4 s0 = *reinterpret_cast<const LK_LOCAL u32x4 *>(scr + 104), s1 = *reinterpret_cast<const LK_LOCAL u32x4 *>(scr + 108);
    const uint32_t pb[8] = { s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3] };
    float sum = 0.f;
#pragma unroll
    for (int r = 0; r < MAXK; ++r) { sum = sum + __builtin_bit_cast(float, pb[r]); }
    sum = sum > 6.103515625e-5f ? sum : 6.103515625e-5f;
    if (lane < MAXK) {
        const float pl = __builtin_bit_cast(float, scr[104 + lane]);
        sel_out[lane] = (int) scr[96 + lane];
        w_out[lane] = pl / sum * scale;
    }
    return true;
}

// the same from the lane's 4 logits; probs_out (optional) receives the n_exp probabilities
__device__ __forceinline__ void select_token(const float (&lg)[4], const float (&bias)[4], int n_exp, int n_group, int topk_group, int topk,
                                             float scale, float * scr, int * sel_out, float * w_out, float * probs_out,
                                             int keep, float renorm) {
    const int lane = lane_id();
    float p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = 4 * lane + j;
        p[j] = 0.f;
        if (e < n_exp) {
            p[j] = det_sigmoid(lg[j]);
            if (probs_out) { gptr(probs_out)[e] = p[j]; }
        }
    }
    select_token_p(p, bias, n_exp, n_group, topk_group, topk, scale, scr, sel_out, w_out, keep, renorm);
}

// --share-experts keep (src/server_core_fused.cpp:798-806) by one wave over n rows, in row order. Row i's topk picks
// (expert, weight) are sel8 / w8 [i * topk ..] in pick order; each row keeps its own min(2, ke) heaviest (weight
// descending, equal weights in pick order), then, in that weight order, its other picks whose expert is in the set U,
// then its remaining picks, each of which joins U as it is taken; renorm > 0 rescales the kept weights by renorm / sw
// with sw their fp32 sum in kept order (when sw > 1e-6). Outputs [i * ke ..] in kept order may alias sel8 / w8 (ke <=
// topk: row i is read whole before it is written, and later rows are never overwritten). U: 8 words of 32 expert bits
// (n_exp <= 256), filled here from every row's own picks when init, else given.
template <class SI, class SF, class DI, class DF, class PU>
__device__ __noinline__ void keep_share_rows(SI sel8, SF w8, int n, int topk, int ke, float renorm, DI sel_out, DF w_out, PU U, bool init) {
#pragma clang fp contract(off)
    const int lane = lane_id(), own = ke < 2 ? ke : 2;
    const bool act = lane < topk;
    auto rank_of = [&](float wv) {
        int r = 0;
        for (int j = 0; j < topk; ++j) {
            const float o = __builtin_bit_cast(float, rdlane(__builtin_bit_cast(uint32_t, wv), j));
            r += (o > wv || (o == wv && j < lane)) ? 1 : 0;
        }
        return r;
    };
    auto visible = [&]() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront"); __builtin_amdgcn_s_waitcnt(0); __builtin_amdgcn_wave_barrier(); };
    if (init) {
        if (lane < 8) { U[lane] = 0u; }
        visible();
        for (int i = 0; i < n; ++i) {
            const int e = act ? sel8[i * topk + lane] : 0;
            const float wv = act ? w8[i * topk + lane] : 0.f;
            const int r = rank_of(wv);
            if (act && r < own) { __hip_atomic_fetch_or(&U[(e >> 5) & 7], 1u << (e & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT); }
        }
        visible();
    }
    for (int i = 0; i < n; ++i) {
        const int e = act ? sel8[i * topk + lane] : 0;
        const float wv = act ? w8[i * topk + lane] : 0.f;
        const int r = rank_of(wv);
        const bool inU = act && ((U[(e >> 5) & 7] >> (e & 31)) & 1u);
        // phase 1: the row's other picks whose expert U holds, by rank; phase 2 (only if phase 1 leaves slots): the rest
        const bool c1 = act && r >= own && inU;
        const bool c2 = act && r >= own && !inU;
        const uint64_t m1 = __ballot(c1), m2 = __ballot(c2);
        int p1 = 0, p2 = 0;   // candidates of the same phase ranked above this lane's pick
        for (int j = 0; j < topk; ++j) {
            const int rj = (int) rdlane((uint32_t) r, j);
            p1 += ((m1 >> j) & 1) && rj < r ? 1 : 0;
            p2 += ((m2 >> j) & 1) && rj < r ? 1 : 0;
        }
        const int n1 = __popcll(m1), t1 = n1 < ke - own ? n1 : ke - own;
        const bool take1 = c1 && p1 < ke - own;
        const bool take2 = c2 && own + t1 + p2 < ke;
        const int pos = !act ? -1 : r < own ? r : take1 ? own + p1 : take2 ? own + t1 + p2 : -1;
        float f = 1.f; bool rescale = false;
        if (renorm > 0.f) {
            float sw = 0.0f;
            for (int q = 0; q < ke; ++q) { sw = sw + __builtin_bit_cast(float, rdlane(__builtin_bit_cast(uint32_t, wv), first_lane(pos == q))); }
            if (sw > 1e-6f) { f = renorm / sw; rescale = true; }
        }
        visible();   // the whole row is read before any of it is written (in place)
        if (pos >= 0) { sel_out[i * ke + pos] = e; w_out[i * ke + pos] = rescale ? wv * f : wv; }
        if (take2) { __hip_atomic_fetch_or(&U[(e >> 5) & 7], 1u << (e & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT); }
        visible();
    }
}

}  // namespace lk
