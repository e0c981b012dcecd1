// kq_gemm.hip -- K-quant matrices (the real shards' formats: routed down Q2_K / Q3_K, shared expert Q5_K / Q5_K /
// Q6_K) on the matrix cores at prefill sizes.
//
// Reference: the K-quant mat-vecs of the wide pass (tc_matvec<F_Q2K/F_Q3K/F_Q5K/F_Q6K>, src/fused_layer.cu:102-158,
// 203-254, launched at 520-524 and 541-550). The arithmetic is ggml_vec_dot_q{2,3,5,6}_K_q8_K's as the K-quant
// mat-vec (kquant.hip) restates it, and the outputs are bit-identical to that kernel's: per block the exact integer
// sums isum = sum_j sc_j sum_i q_i x_i (q the stored value minus its offset: Q3_K 4, Q6_K 32) and, for Q2_K / Q5_K,
// summ = sum_j mn_j bsum_j; then over the blocks in order
//   Q2_K         acc += (d8 * d) * isum - (d8 * dmin) * summ
//   Q3_K, Q6_K   acc += (d * d8) * isum
//   Q5_K         acc_s += (d * d8) * isum, acc_m -= (dmin * d8) * summ, result acc_m + acc_s
// with isum and summ rounded to fp32 once.
//
// The integer sums come from v_mfma_f32_16x16x32_f16 chains per 16 x 16 (token, row) tile, the activations being the
// Q8_K integers as fp16 and the weights fp16 integers built exactly: the stored value u's byte is placed in an fp16
// 1024 + u by one byte permute, and fma(1024 + u, sc, -1024 sc) = u * sc is exact whenever |u * sc| <= 2048 (the fma
// rounds once and fp16 holds every integer up to 2048; Q6_K, whose 8-bit scales make -1024 sc overflow fp16, takes
// (1024 + u - 1024) * sc instead). The chains:
//   A    sum u * sc * x   (Q6_K: u's low 4 bits; |u * sc| <= 7 * 32 (Q3_K), 3 * 15 (Q2_K), 31 * 63 (Q5_K), 15 * 128)
//   A2   sum (u >> 4) * sc * x                              (Q6_K only: |.| <= 3 * 128)
//   B    sum v * x, v the sub-block's scale (Q3_K, Q6_K: the offset term) or min (Q2_K, Q5_K)
// and isum = A (Q2_K, Q5_K), A - 4 B (Q3_K), A + 16 A2 - 32 B (Q6_K); summ = B. A chain's products and partial sums
// are integers, so it is exact whatever order the matrix core adds in while every partial sum stays below 2^24: A runs
// over segments of SEG steps of 32 products (Q2_K, Q3_K: the whole block, at most 256 * 224 * 127 < 7.3e6; Q5_K,
// Q6_K: two steps, at most 64 * 1953 * 127 < 1.6e7), A2 and B over the whole block; the segment totals are converted
// to int32 (exactly) and the block sums formed in int32.
//
// Work: as the IQ2_XXS grouped GEMM (moe_prefill.hip): a column is up to 64 dispatch slots of one expert (or of the
// shared expert), an item is (column, 128 rows), one 8-wave workgroup per CU takes the items round-robin. Wave w owns
// one 16-row tile (two spill: the slices' raw bytes are double-buffered in registers); lane (r, g) holds row r of the
// tile and the lane slices 2 g, 2 g + 1 of each block (kquant_device.h's slices, 32 weights each). Step t of lane
// group g covers 8 of them (slice 2 g + t / 4): Q2_K / Q3_K / Q6_K piece t % 4, block weights 128 n + 32 s + 8 jq ..
// + 7 (n = g / 2, s = t % 4, jq = 2 (g % 2) + t / 4); Q5_K half t % 2 of piece (t % 4) / 2, weights
// 64 g + 32 h + 16 k + 8 e .. + 7 (h = (t % 4) / 2, k = t / 4, e = t % 2). The activation operand reads the same 8
// positions, so both operands permute K alike. The column's activations go block by block from memory into LDS
// (direct loads, double-buffered); the next block's weight bytes are in flight while a block computes.
#include "kquant_device.h"
#include "moe_kernels.h"
#include <type_traits>

namespace lk {

namespace {

typedef _Float16 kh8 __attribute__((ext_vector_type(8)));
typedef _Float16 kh2 __attribute__((ext_vector_type(2)));
typedef float kf4 __attribute__((ext_vector_type(4)));

constexpr int KG_W = 8, KG_NT = KG_W * 64;   // waves / threads per workgroup
constexpr int KG_ROWS = KG_W * 16;           // rows per item: one 16-row tile per wave
constexpr int KG_NTM = 4;                    // 16-token tiles per column at most
// LDS: two activation buffers of 64 token rows x 512 B (each row's 16-byte chunks XOR-swizzled by the row)
constexpr int KG_TILE = 16 * 512, KG_BUF = KG_NTM * KG_TILE, KG_LDS = 2 * KG_BUF;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t kg_rsrc(const void * p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short) 0, (int) bytes, 0x00020000);
}
__device__ __forceinline__ const uint8_t * kg_uniform(const uint8_t * p) {
    const uint64_t v = (uint64_t) p;
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) (v >> 32));
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) v);
    return (const uint8_t *) (((uint64_t) hi << 32) | (uint64_t) lo);
}
// 16 bytes per lane from a buffer straight into LDS (lane L at dst + 16 L); the builtin exists for the device pass only
__device__ __forceinline__ void kg_lds16(__amdgpu_buffer_rsrc_t r, LK_LOCAL uint8_t * dst, uint32_t voff, uint32_t soff) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LK_LOCAL void *) dst, 16, voff, soff, 0, 0);
#else
    (void) r; (void) dst; (void) voff; (void) soff;
#endif
}

// 8 weights sc * u (u the bytes of u0, u1) as fp16, exact for |u * sc| <= 2048: byte b -> fp16 bits 0x6400 | b =
// 1024 + b, then fma(1024 + b, sc, -1024 sc) = b * sc (the exact value is an fp16 integer, and the fma rounds once).
// The constant -1024 sc is an fp16 for |sc| <= 63; BIG (|sc| up to 128, Q6_K) subtracts 1024 first, then multiplies.
template <bool BIG> __device__ __forceinline__ kh8 kg_weights(uint32_t u0, uint32_t u1, kh2 s2, kh2 c2) {
    const uint32_t p[4] = { __builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u),
                            __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u) };
    kh8 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        kh2 h;
        if constexpr (BIG) { const kh2 m = { (_Float16) -1024.f, (_Float16) -1024.f }; h = (__builtin_bit_cast(kh2, p[i]) + m) * s2; }
        else { h = __builtin_elementwise_fma(__builtin_bit_cast(kh2, p[i]), s2, c2); }
        w[2 * i] = h[0]; w[2 * i + 1] = h[1];
    }
    return w;
}

template <int F> struct KgFmt {
    static constexpr bool Q5 = F == KF_Q5K, Q6 = F == KF_Q6K;
    static constexpr bool MINS = F == KF_Q2K || F == KF_Q5K;   // summ terms
    static constexpr int SEG = (Q5 || Q6) ? 2 : 8;              // steps per exact segment of chain A
    static constexpr bool NT4 = !(Q5 || Q6);   // four token tiles per pass (Q5_K / Q6_K: two, a 64-slot column in two passes; four spill)
};

template <int F, int NB>
__global__ void __launch_bounds__(KG_NT, 1) k_kq_gemm(const PrefillArgs a) {
#pragma clang fp contract(off)
    using Fm = KgFmt<F>;
    constexpr int BS = kbytes<F>();
    constexpr uint32_t ROWB = (uint32_t) (NB * BS);   // bytes of a row
    static_assert(NB % 2 == 0, "two blocks per pipeline trip");
    extern __shared__ __attribute__((aligned(16))) uint8_t kg_dyn[];
    LK_LOCAL uint8_t * lds = (LK_LOCAL uint8_t *) kg_dyn;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = lane_id();
    const int r = lane & 15, g = lane >> 4;
    const int col0 = a.col0, ncols = (a.col1 > 0 ? a.col1 : *gptr(a.ncols)) - col0;
    const int nrg = a.R / KG_ROWS;
    const uint32_t mbytes = (uint32_t) a.R * ROWB;   // one matrix

    for (int it = blockIdx.x; it < ncols * nrg; it += gridDim.x) {
        const int col = col0 + it / nrg, rg = it % nrg;
        const u32x4 cv = *(const LK_GLOBAL u32x4 *) (a.cols + col);
        const bool routed = (int) cv.x >= 0;
        const int e = (int) cv.w;
        const __amdgpu_buffer_rsrc_t rb = kg_rsrc(a.bh, 0x7fffffff), rd = kg_rsrc(a.bd, 0x7fffffff);
        const uint8_t * W = routed ? a.w[0] + (size_t) e * a.estride : a.sh[0];
        Src src;
        src.rs = kg_rsrc(kg_uniform(W), mbytes);
        src.vb = (uint32_t) r * ROWB;
        src.so = (uint32_t) (rg * KG_ROWS + wave * 16) * ROWB;
        // one pass over the item's weights for the slots sb .. sb + sc - 1 (sc <= 16 NT)
        auto run_item = [&](auto ntc, const int sb, const int sc) {
            constexpr int NT = decltype(ntc)::value;
            const int ar0 = sb - a.arow0;   // the first activation row
            const uint32_t oX = (uint32_t) (ar0 + (lane < sc ? lane : 0)) * (NB * 4);   // lane n: token n's block scales
            // activation rows: wave w copies token rows RW w + 2 i + (lane / 32), lane L < 32 of a row taking the row's
            // chunk pf_swz(L ^ (row % 16)), so chunk c sits at slot pf_swz(c) ^ (row % 16)
            constexpr int RW = 16 * NT / KG_W, NI = RW / 2;
            static_assert(RW % 2 == 0, "two token rows per copy instruction");
            uint32_t ob[NI];
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int row = RW * wave + 2 * i + (lane >> 5);
                ob[i] = (uint32_t) (ar0 + (row < sc ? row : 0)) * (NB * QK * 2) + pf_swz((uint32_t) ((lane & 31) ^ (row & 15))) * 16;
            }
            auto load_b = [&](int j, int buf) -> float {
                LK_LOCAL uint8_t * dst = lds + buf * KG_BUF;
#pragma unroll
                for (int i = 0; i < NI; ++i) { kg_lds16(rb, dst + (RW * wave + 2 * i) * 512, ob[i], j * (QK * 2)); }
                return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rd, oX, j * 4, 0));
            };
            auto load_w = [&](int j, Raw<F> (&w)[2]) {
                Src s = src; s.vb += (uint32_t) (j * BS);
                load_raw<F>(s, 2 * g, w[0]); load_raw<F>(s, 2 * g + 1, w[1]);
            };
            kf4 acc[NT], accm[NT];
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) { acc[tt] = (kf4) { 0.f, 0.f, 0.f, 0.f }; accm[tt] = acc[tt]; }
            // one block: the lane's two slices decoded just before their four steps, the chains of every token tile,
            // the block sums in int32, then the fold
            auto block = [&](const Raw<F> (&w)[2], int buf, float dxl) {
                kf4 ca[NT], ca2[NT], cb[NT];
                int is[NT][4], sm[NT][4];
#pragma unroll
                for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) { is[tt][i] = 0; sm[tt][i] = 0; }
                }
                float dd = 0.f, dm = 0.f;
                const uint32_t base = (uint32_t) (size_t) (lds + buf * KG_BUF) + (uint32_t) r * 512;
                const kf4 z = { 0.f, 0.f, 0.f, 0.f };
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    Chunk ck;
                    decode<F>(w[k], 2 * g + k, ck);
                    if (k == 0) { dd = ck.d; dm = ck.dmin; }
#pragma unroll
                    for (int s4 = 0; s4 < 4; ++s4) {
                        const int t = 4 * k + s4;
                        int ch, p, wi;   // 16-byte chunk of the step's K positions, scale / min index, first word
                        if constexpr (Fm::Q5) { const int h = s4 >> 1, ee = s4 & 1; ch = 8 * g + 4 * h + 2 * k + ee; p = h; wi = 4 * h + 2 * ee; }
                        else { ch = 16 * (g >> 1) + 4 * s4 + 2 * (g & 1) + k; p = s4; wi = 2 * s4; }
                        kh8 x[NT];
#pragma unroll
                        for (int tt = 0; tt < NT; ++tt) {
                            x[tt] = __builtin_bit_cast(kh8, *(const LK_LOCAL u32x4 *) (size_t) (base + tt * KG_TILE + ((pf_swz((uint32_t) ch) ^ (uint32_t) r) << 4)));
                        }
                        const int scv = ck.sc[p];
                        const _Float16 sf = (_Float16) scv, cf = (_Float16) (Fm::Q6 ? 0.f : -1024.f * (float) scv);
                        const kh2 s2 = { sf, sf }, c2 = { cf, cf };
                        uint32_t u0 = ck.u[wi], u1 = ck.u[wi + 1];
                        if constexpr (Fm::Q6) { u0 &= 0x0F0F0F0Fu; u1 &= 0x0F0F0F0Fu; }
                        const kh8 wv = kg_weights<Fm::Q6>(u0, u1, s2, c2);
                        const _Float16 vf = (_Float16) (Fm::MINS ? ck.mn[p] : scv);
                        const kh8 vv = { vf, vf, vf, vf, vf, vf, vf, vf };
                        const bool seg0 = t % Fm::SEG == 0;
#pragma unroll
                        for (int tt = 0; tt < NT; ++tt) {
                            ca[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[tt], wv, seg0 ? z : ca[tt], 0, 0, 0);
                            cb[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[tt], vv, t == 0 ? z : cb[tt], 0, 0, 0);
                        }
                        if constexpr (Fm::Q6) {
                            const kh8 wh = kg_weights<true>((ck.u[wi] >> 4) & 0x03030303u, (ck.u[wi + 1] >> 4) & 0x03030303u, s2, c2);
#pragma unroll
                            for (int tt = 0; tt < NT; ++tt) {
                                ca2[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[tt], wh, t == 0 ? z : ca2[tt], 0, 0, 0);
                            }
                        }
                        if (t % Fm::SEG == Fm::SEG - 1) {   // the segment's exact total into the int32 block sum
#pragma unroll
                            for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
                                for (int i = 0; i < 4; ++i) { is[tt][i] += (int) ca[tt][i]; }
                            }
                        }
                    }
                }
#pragma unroll
                for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int b = (int) cb[tt][i];
                        if constexpr (F == KF_Q3K) { is[tt][i] -= 4 * b; }
                        else if constexpr (Fm::Q6) { is[tt][i] += 16 * (int) ca2[tt][i] - 32 * b; }
                        else { sm[tt][i] = b; }
                    }
                }
                // fold in block order: the scale of token 16 tt + 4 g + i comes from the lane that loaded it
#pragma unroll
                for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float d8 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * (16 * tt + 4 * g + i), __builtin_bit_cast(int, dxl)));
                        const float fi = (float) is[tt][i];
                        if constexpr (F == KF_Q2K) {
                            acc[tt][i] = acc[tt][i] + ((d8 * dd) * fi - (d8 * dm) * (float) sm[tt][i]);
                        } else if constexpr (Fm::Q5) {
                            acc[tt][i] = acc[tt][i] + (dd * d8) * fi;
                            accm[tt][i] = accm[tt][i] - (dm * d8) * (float) sm[tt][i];
                        } else {
                            acc[tt][i] = acc[tt][i] + (dd * d8) * fi;
                        }
                    }
                }
            };
            // pipeline: the next block's weight bytes (registers) and activations (the other LDS buffer) are loaded
            // while a block computes; buffer (j + 1) % 2 was last read in block j - 1, before its barrier
            Raw<F> w0[2], w1[2];
            load_w(0, w0);
            float dxl = load_b(0, 0);
            __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): block 0's activations are in LDS
            __syncthreads();
            auto step = [&](int j, const Raw<F> (&cur)[2], Raw<F> (&nxt)[2]) {
                const float dcur = dxl;
                const int jn = j + 1 < NB ? j + 1 : NB - 1;   // the last step reloads its own block (unread)
                dxl = load_b(jn, (j + 1) & 1);
                load_w(jn, nxt);
                __builtin_amdgcn_sched_barrier(0);
                block(cur, j & 1, dcur);
                __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): block j + 1's activations have landed in LDS
                __builtin_amdgcn_s_barrier();
            };
#pragma unroll 1
            for (int j = 0; j < NB; j += 2) { step(j, w0, w1); step(j + 1, w1, w0); }
            const int row = rg * KG_ROWS + wave * 16 + r;
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int n = 16 * tt + 4 * g + i;
                    if (n < sc) { a.out[(size_t) (sb - a.orow0 + n) * a.R + row] = Fm::Q5 ? accm[tt][i] + acc[tt][i] : acc[tt][i]; }
                }
            }
        };
        const int sb = (int) cv.y, sc = (int) cv.z;
        if (sc > 32) {
            if constexpr (Fm::NT4) { run_item(std::integral_constant<int, 4>{}, sb, sc); }
            else { run_item(std::integral_constant<int, 2>{}, sb, 32); run_item(std::integral_constant<int, 2>{}, sb + 32, sc - 32); }
        } else if (sc > 16) { run_item(std::integral_constant<int, 2>{}, sb, sc); }
        else { run_item(std::integral_constant<int, 1>{}, sb, sc); }
        __syncthreads();   // the LDS buffers are refilled by the next item
    }
}

template <int F, int NB> hipError_t kg_setup() {
    return hipFuncSetAttribute((const void *) k_kq_gemm<F, NB>, hipFuncAttributeMaxDynamicSharedMemorySize, KG_LDS);
}
template <int F, int NB> void kg_go(const PrefillArgs & a, int grid, hipStream_t st) { k_kq_gemm<F, NB><<<grid, KG_NT, KG_LDS, st>>>(a); }

}  // namespace

hipError_t kq_gemm_init() {
    hipError_t e = kg_setup<KF_Q2K, 8>();
    if (e == hipSuccess) { e = kg_setup<KF_Q3K, 8>(); }
    if (e == hipSuccess) { e = kg_setup<KF_Q6K, 8>(); }
    if (e == hipSuccess) { e = kg_setup<KF_Q5K, 28>(); }
    return e;
}

hipError_t launch_kq_gemm(const PrefillArgs & a, int fmt, int grid, hipStream_t st) {
    const int nb = a.K / QK;
    const bool down = nb == 8 && (fmt == KF_Q2K || fmt == KF_Q3K || fmt == KF_Q6K), gu = nb == 28 && fmt == KF_Q5K;
    if (grid < 1 || !a.cols || !a.ncols || !a.bh || !a.bd || !a.out || a.K % QK || a.R % KG_ROWS || !(down || gu) || a.col0 < 0 ||
        ((reinterpret_cast<uintptr_t>(a.w[0]) | reinterpret_cast<uintptr_t>(a.sh[0]) | a.estride) & 3u) ||
        (uint64_t) a.R * nb * kq_block_bytes(fmt) >= 0x7fffffffull) {
        return hipErrorInvalidValue;
    }
    if (fmt == KF_Q2K) { kg_go<KF_Q2K, 8>(a, grid, st); }
    else if (fmt == KF_Q3K) { kg_go<KF_Q3K, 8>(a, grid, st); }
    else if (fmt == KF_Q6K) { kg_go<KF_Q6K, 8>(a, grid, st); }
    else { kg_go<KF_Q5K, 28>(a, grid, st); }
    return hipGetLastError();
}

}  // namespace lk
