// kq_gemm.hip -- the routed down in Q2_K / Q3_K (the real shards' formats) on the matrix cores at prefill sizes.
//
// Reference: the K-quant down of the wide pass (tc_matvec<F_Q2K/F_Q3K>, src/fused_layer.cu:203-254, 541-550). The
// arithmetic is ggml_vec_dot_q{2,3}_K_q8_K's as the K-quant mat-vec (kquant.hip) restates it, and the outputs are
// bit-identical to that kernel's:
//   per block, the exact integer sums isum = sum_j sc_j sum_i q_i x_i (Q3_K: q = u - 4, u the stored 3-bit value) and,
//   for Q2_K, summ = sum_j mn_j bsum_j; then, over the blocks in order, acc += term with
//   Q2_K term = (d8 * d) * isum - (d8 * dmin) * summ, Q3_K term = (d * d8) * isum.
// The integer sums come from two v_mfma_f32_16x16x32_f16 chains per 16 x 16 (token, row) tile over a block's 8 K-steps:
//   * chain A with the weights sc_j * u (|w| <= 31 * 7 < 2^8), each built exactly as fma(1024 + u, sc, -1024 sc) from
//     the u byte placed in an fp16 1024 + u by one byte permute (fp16 holds every integer below 2048);
//   * chain B with the sub-block's constant v_j: Q3_K sc_j, so isum = A - 4 B (the -4 of every stored value); Q2_K
//     mn_j, so summ = B.
// The activations are the Q8_K integers as fp16. Every product and partial sum is an integer below 2^24 (chain A at
// most 256 * 224 * 127 < 7.3e6 in magnitude), so each chain's total is exact whatever order the matrix core adds in,
// and A - 4 B is exact too.
//
// Work: as the IQ2_XXS grouped GEMM (moe_prefill.hip): a column is up to 64 dispatch slots of one expert, an item is
// (column, 128 rows), one 8-wave workgroup per CU takes the items round-robin. Wave w owns one 16-row tile (two
// spill: the slices' raw bytes are double-buffered in registers); lane (r, g) holds row r of the tile and the lane
// slices 2 g, 2 g + 1 of each block (kquant_device.h's slices: 32 weights
// each, 4 pieces of 8 sharing one sub-block scale). Step t of lane group g is piece t % 4 of slice 2 g + t / 4, i.e.
// block weights 128 n + 32 s + 8 jq .. + 7 (n = g / 2, s = t % 4, jq = 2 (g % 2) + t / 4); the activation operand
// reads the same 8 positions, so both operands permute K alike. The column's activations go block by block from
// memory into LDS (direct loads, double-buffered); the next block's weight bytes are in flight while a block computes.
#include "kquant_device.h"
#include "moe_kernels.h"
#include <type_traits>

namespace lk {

namespace {

typedef _Float16 kh8 __attribute__((ext_vector_type(8)));
typedef _Float16 kh2 __attribute__((ext_vector_type(2)));
typedef float kf4 __attribute__((ext_vector_type(4)));

constexpr int KG_W = 8, KG_NT = KG_W * 64;   // waves / threads per workgroup
constexpr int KG_RGI = 1;                    // 16-row tiles per wave
constexpr int KG_ROWS = KG_W * 16 * KG_RGI;  // rows per item (128)
constexpr int KG_NTM = 4;                    // 16-token tiles per column at most
constexpr int KG_NB = 8;                     // blocks per row (K = 2048)
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

// 8 weights sc * u (u the bytes of u0, u1) as fp16, exact: byte b -> fp16 bits 0x6400 | b = 1024 + b, then
// fma(1024 + b, sc, -1024 sc) = b * sc (the exact value is an fp16 integer, and the fma rounds once)
__device__ __forceinline__ kh8 kg_weights(uint32_t u0, uint32_t u1, kh2 s2, kh2 c2) {
    const uint32_t p[4] = { __builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u),
                            __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u) };
    kh8 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const kh2 h = __builtin_elementwise_fma(__builtin_bit_cast(kh2, p[i]), s2, c2);
        w[2 * i] = h[0]; w[2 * i + 1] = h[1];
    }
    return w;
}

template <int F>
__global__ void __launch_bounds__(KG_NT, 1) k_kq_gemm(const PrefillArgs a) {
#pragma clang fp contract(off)
    static_assert(F == KF_Q2K || F == KF_Q3K, "the routed down formats");
    constexpr int BS = kbytes<F>();
    constexpr uint32_t ROWB = (uint32_t) (KG_NB * BS);   // bytes of a row
    extern __shared__ __attribute__((aligned(16))) uint8_t kg_dyn[];
    LK_LOCAL uint8_t * lds = (LK_LOCAL uint8_t *) kg_dyn;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = lane_id();
    const int r = lane & 15, g = lane >> 4;
    const int ncols = *gptr(a.ncols);
    const int nrg = a.R / KG_ROWS;
    const uint32_t mbytes = (uint32_t) a.R * ROWB;   // one expert's matrix

    for (int it = blockIdx.x; it < ncols * nrg; it += gridDim.x) {
        const int col = it / nrg, rg = it - col * nrg;
        const u32x4 cv = *(const LK_GLOBAL u32x4 *) (a.cols + col);
        if ((int) cv.x < 0) { continue; }   // the shared expert's columns: not this kernel's (its down runs apart)
        const int sb = (int) cv.y, sc = (int) cv.z, e = (int) cv.w;
        const __amdgpu_buffer_rsrc_t rb = kg_rsrc(a.bh, 0x7fffffff), rd = kg_rsrc(a.bd, 0x7fffffff);
        const __amdgpu_buffer_rsrc_t rw = kg_rsrc(kg_uniform(a.w[0] + (size_t) e * a.estride), mbytes);
        // the lane's weight rows: tile ti = rows rg * KG_ROWS + (KG_RGI w + ti) * 16 + r
        Src src[KG_RGI];
#pragma unroll
        for (int ti = 0; ti < KG_RGI; ++ti) {
            src[ti].rs = rw;
            src[ti].vb = (uint32_t) r * ROWB;
            src[ti].so = (uint32_t) (rg * KG_ROWS + (wave * KG_RGI + ti) * 16) * ROWB;
        }
        const uint32_t oX = (uint32_t) (sb + (lane < sc ? lane : 0)) * (KG_NB * 4);   // lane n: token n's block scales
        auto run_item = [&](auto ntc) {
            constexpr int NT = decltype(ntc)::value;
            // activation rows: wave w copies token rows RW w + 2 i + (lane / 32), lane L < 32 of a row taking the row's
            // chunk L ^ (row % 16)
            constexpr int RW = 16 * NT / KG_W, NI = RW / 2;
            static_assert(RW % 2 == 0, "two token rows per copy instruction");
            uint32_t ob[NI];
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int row = RW * wave + 2 * i + (lane >> 5);
                ob[i] = (uint32_t) (sb + (row < sc ? row : 0)) * (KG_NB * QK * 2) + (uint32_t) ((lane & 31) ^ (row & 15)) * 16;
            }
            auto load_b = [&](int j, int buf) -> float {
                LK_LOCAL uint8_t * dst = lds + buf * KG_BUF;
#pragma unroll
                for (int i = 0; i < NI; ++i) { kg_lds16(rb, dst + (RW * wave + 2 * i) * 512, ob[i], j * (QK * 2)); }
                return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rd, oX, j * 4, 0));
            };
            auto load_w = [&](int j, Raw<F> (&w)[KG_RGI][2]) {
#pragma unroll
                for (int ti = 0; ti < KG_RGI; ++ti) {
                    Src s = src[ti]; s.vb += (uint32_t) (j * BS);
                    load_raw<F>(s, 2 * g, w[ti][0]); load_raw<F>(s, 2 * g + 1, w[ti][1]);
                }
            };
            kf4 acc[KG_RGI][NT];
#pragma unroll
            for (int ti = 0; ti < KG_RGI; ++ti) {
#pragma unroll
                for (int tt = 0; tt < NT; ++tt) { acc[ti][tt] = (kf4) { 0.f, 0.f, 0.f, 0.f }; }
            }
            // one block: decode the lane's two slices of each tile, run the two chains of every (tile, token tile), fold
            auto block = [&](const Raw<F> (&w)[KG_RGI][2], int buf, float dxl) {
                kf4 ca[KG_RGI][NT], cb[KG_RGI][NT];
                float dd[KG_RGI], dm[KG_RGI];
                const uint32_t base = (uint32_t) (size_t) (lds + buf * KG_BUF) + (uint32_t) r * 512;
#pragma unroll
                for (int k = 0; k < 2; ++k) {   // slice 2 g + k of each tile, decoded just before its four steps
                    Chunk ck[KG_RGI];
#pragma unroll
                    for (int ti = 0; ti < KG_RGI; ++ti) {
                        decode<F>(w[ti][k], 2 * g + k, ck[ti]);
                        if (k == 0) { dd[ti] = ck[ti].d; dm[ti] = ck[ti].dmin; }
                    }
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const int t = 4 * k + s;
                        const int ch = 16 * (g >> 1) + 4 * s + 2 * (g & 1) + k;   // the step's 8 K positions, in 16-byte chunks
                        kh8 x[NT];
#pragma unroll
                        for (int tt = 0; tt < NT; ++tt) {
                            x[tt] = __builtin_bit_cast(kh8, *(const LK_LOCAL u32x4 *) (size_t) (base + tt * KG_TILE + ((uint32_t) (ch ^ r) << 4)));
                        }
#pragma unroll
                        for (int ti = 0; ti < KG_RGI; ++ti) {
                            const Chunk & c = ck[ti];
                            const _Float16 sf = (_Float16) c.sc[s], cf = (_Float16) (-1024.f * (float) c.sc[s]);
                            const kh2 s2 = { sf, sf }, c2 = { cf, cf };
                            const kh8 wv = kg_weights(c.u[2 * s], c.u[2 * s + 1], s2, c2);
                            const _Float16 vf = (_Float16) (F == KF_Q3K ? c.sc[s] : c.mn[s]);
                            const kh8 vv = { vf, vf, vf, vf, vf, vf, vf, vf };
                            const kf4 z = { 0.f, 0.f, 0.f, 0.f };
#pragma unroll
                            for (int tt = 0; tt < NT; ++tt) {
                                ca[ti][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[tt], wv, t == 0 ? z : ca[ti][tt], 0, 0, 0);
                                cb[ti][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[tt], vv, t == 0 ? z : cb[ti][tt], 0, 0, 0);
                            }
                        }
                    }
                }
                // fold in block order: the scale of token 16 tt + 4 g + i comes from the lane that loaded it
                float dx[NT][4];
#pragma unroll
                for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        dx[tt][i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * (16 * tt + 4 * g + i), __builtin_bit_cast(int, dxl)));
                    }
                }
#pragma unroll
                for (int ti = 0; ti < KG_RGI; ++ti) {
                    const float d = dd[ti], dmin = dm[ti];
#pragma unroll
                    for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            float term;
                            if constexpr (F == KF_Q2K) {
                                term = (dx[tt][i] * d) * ca[ti][tt][i] - (dx[tt][i] * dmin) * cb[ti][tt][i];
                            } else {
                                term = (d * dx[tt][i]) * (ca[ti][tt][i] - 4.f * cb[ti][tt][i]);
                            }
                            acc[ti][tt][i] = acc[ti][tt][i] + term;
                        }
                    }
                }
            };
            // pipeline: the next block's weight bytes (registers) and activations (the other LDS buffer) are loaded
            // while a block computes; buffer (j + 1) % 2 was last read in block j - 1, before its barrier
            Raw<F> w0[KG_RGI][2], w1[KG_RGI][2];
            load_w(0, w0);
            float dxl = load_b(0, 0);
            __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): block 0's activations are in LDS
            __syncthreads();
            auto step = [&](int j, const Raw<F> (&cur)[KG_RGI][2], Raw<F> (&nxt)[KG_RGI][2]) {
                const float dcur = dxl;
                const int jn = j + 1 < KG_NB ? j + 1 : KG_NB - 1;   // the last step reloads its own block (unread)
                dxl = load_b(jn, (j + 1) & 1);
                load_w(jn, nxt);
                __builtin_amdgcn_sched_barrier(0);
                block(cur, j & 1, dcur);
                __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): block j + 1's activations have landed in LDS
                __builtin_amdgcn_s_barrier();
            };
#pragma unroll 1
            for (int j = 0; j < KG_NB; j += 2) { step(j, w0, w1); step(j + 1, w1, w0); }
#pragma unroll
            for (int ti = 0; ti < KG_RGI; ++ti) {
                const int row = rg * KG_ROWS + (wave * KG_RGI + ti) * 16 + r;
#pragma unroll
                for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int n = 16 * tt + 4 * g + i;
                        if (n < sc) { a.out[(size_t) (sb + n) * a.R + row] = acc[ti][tt][i]; }
                    }
                }
            }
        };
        if (sc > 32) { run_item(std::integral_constant<int, 4>{}); }
        else if (sc > 16) { run_item(std::integral_constant<int, 2>{}); }
        else { run_item(std::integral_constant<int, 1>{}); }
        __syncthreads();   // the LDS buffers are refilled by the next item
    }
}

}  // namespace

hipError_t kq_gemm_init() {
    hipError_t e = hipFuncSetAttribute((const void *) k_kq_gemm<KF_Q2K>, hipFuncAttributeMaxDynamicSharedMemorySize, KG_LDS);
    if (e == hipSuccess) { e = hipFuncSetAttribute((const void *) k_kq_gemm<KF_Q3K>, hipFuncAttributeMaxDynamicSharedMemorySize, KG_LDS); }
    return e;
}

hipError_t launch_kq_gemm(const PrefillArgs & a, int fmt, int grid, hipStream_t st) {
    if (grid < 1 || !a.cols || !a.ncols || !a.bh || !a.bd || !a.out || !a.w[0] || a.K != KG_NB * QK || a.R % KG_ROWS ||
        (fmt != KF_Q2K && fmt != KF_Q3K) || (reinterpret_cast<uintptr_t>(a.w[0]) & 3u) || (a.estride & 3u) ||
        (uint64_t) a.R * KG_NB * kq_block_bytes(fmt) >= 0x7fffffffull) {
        return hipErrorInvalidValue;
    }
    if (fmt == KF_Q2K) { k_kq_gemm<KF_Q2K><<<grid, KG_NT, KG_LDS, st>>>(a); }
    else { k_kq_gemm<KF_Q3K><<<grid, KG_NT, KG_LDS, st>>>(a); }
    return hipGetLastError();
}

}  // namespace lk
