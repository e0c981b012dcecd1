// moe_prefill.hip -- the grouped IQ2_XXS x Q8_K expert GEMMs of a prefill batch on the matrix cores.
//
// Reference: fl_wide_moe (src/fused_layer.cu:540-561) runs tc_matvec<F_IQ2> (:178-202) per arena batch of <= 72 slots
// of <= 8 rows each with mma.m16n8k32 s8 tiles, then swiglu_q8 (:334-341) and the down pass; the semantics are ggml's
// mul_mat_id over IQ2_XXS x Q8_K (ggml_vec_dot_iq2_xxs_q8_K per output). Here one launch covers every expert of the
// layer:
//   * A column is up to 64 dispatch slots (PF_TOK) of one expert (the shared expert's slots P .. P + n - 1 included); an item is
//     (column, 256 or 512 rows). The workgroups (one per CU: the tables fill most of the LDS) take the items round-robin.
//   * The weights are dequantised once per item into fp16 MFMA operands: lane (r, g) of a wave owns row r of a 16-row
//     tile and the 16-byte chunk g of each block (sub-blocks 2g, 2g + 1, both with their scale nibbles), so it builds
//     w = sign * grid * (2 nibble + 1) from two replicated LDS tables (fp16 codebook words, fp16 sign masks) and one
//     packed fp16 multiply per two weights. Every w is an integer of magnitude <= 43 * 31, exact in fp16.
//   * The column's activations (the Q8_K integers as fp16, exact) are copied block by block into LDS with direct
//     global->LDS loads, double-buffered; v_mfma_f32_16x16x32_f16 then forms, per 256-value block, the block sum
//     bsum = sum_ib (2 s_ib + 1) sum_k g s q over a 16-token x 16-row tile, as two chains of four MFMA steps: steps
//     0-3 cover sub-blocks 0, 2, 4, 6 (one per lane group) and steps 4-7 the odd ones. No codebook entry's 8 bytes
//     sum above 203, so a chain's products and every partial sum are integers of magnitude at most
//     16 * 203 * 31 * 127 = 12,787,376 < 2^24: each chain total is exact, whatever order the matrix core adds in. The
//     block sum is then one fp32 addition of the two exact totals, i.e. the exact integer rounded to nearest even --
//     exactly ggml's (float) of its int32 block sum, also where |bsum| exceeds 2^24 (up to 25.6 M).
//   * Each output then advances in block order, y += (d_w * d_x) * bsum, and ends * 0.125: the fp32 operations and their
//     order are those of ggml_vec_dot_iq2_xxs_q8_K, so every output is bit-identical to the CPU checker's.
//   * Gate/up tiles write h = silu(g) * u per slot; down tiles write o per slot (the combine runs after).
// The K index of an MFMA step is permuted consistently in both operands: step t of lane group g covers the 8 values
// 64 g + 8 t .. + 7 of the block, i.e. entry t % 4 of sub-block 2 g + t / 4, which is what the lane's chunk holds.
#include "moe_device.h"
#include "moe_kernels.h"
#include <type_traits>

namespace lk {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int PF_NTM = 4;                    // 16-token MFMA tiles per column at most
constexpr int PF_TOK = 16 * PF_NTM;          // slots per column: the dequantised weights of an item serve all of them
// LDS: fp16 codebook (256 lines x 16 copies x 16 B), fp16 sign masks (128 lines, the 7 stored sign bits), then two
// activation buffers (up to 64 token rows x 512 B, each row's 16-byte chunks XOR-swizzled by the row; the wide kernel's
// fill the 160 KB exactly), then (narrow gate/up) the exchange of g. The tokens' block scales stay in registers (one per
// lane, handed to the lanes that fold them by ds_bpermute).
constexpr int L_PG = 0, L_PS = 65536, L_PB = L_PS + 128 * 256;
constexpr int PB_TILE = 16 * 512;            // one 16-token tile of a buffer (512-byte aligned)
constexpr int PTAB_BYTES = L_PB;             // the table image copied to LDS offset 0

// fp16 table image: line e of the codebook = 16 copies of the 8 fp16 values of grid[e]; line b of the signs = 16
// copies of 8 fp16 sign masks (0x8000 for a negative weight) of the stored sign bits b (0..127) plus parity
__global__ void k_ptab_image(uint32_t * img) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;   // dword index
    if (i >= PTAB_BYTES / 4) { return; }
    const int line = (i * 4) >> 8, word = i & 3;            // 16 B entry copies: the dword inside the entry
    uint32_t v;
    if (i * 4 < L_PS) {
        const uint64_t gv = g_iq2xxs_grid[line];
        const uint32_t b0 = (uint32_t) (gv >> (16 * word)) & 255u, b1 = (uint32_t) (gv >> (16 * word + 8)) & 255u;
        v = (uint32_t) __half_as_ushort(__float2half((float) b0)) | ((uint32_t) __half_as_ushort(__float2half((float) b1)) << 16);
    } else {
        const uint32_t s8 = ksigns8((uint32_t) (line - L_PS / 256));
        v = (((s8 >> (2 * word)) & 1u) << 15) | (((s8 >> (2 * word + 1)) & 1u) << 31);
    }
    img[i] = v;
}
hipError_t build_prefill_tables(uint4 * img, hipStream_t st) {
    k_ptab_image<<<PTAB_BYTES / 4 / 256, 256, 0, st>>>(reinterpret_cast<uint32_t *>(img));
    return hipGetLastError();
}
size_t prefill_table_bytes() { return PTAB_BYTES; }

// Columns: the shared expert's slots first (P + 64 c ..), then every active expert's slots, 64 per column. A column of
// at most 32 slots is narrow (the narrow GEMM takes it), every other one wide; only an expert's last column can be
// narrow. Order: the shared expert's columns (its last one the only narrow one), then the routed wide columns in act
// order, then the routed narrow columns in act order, so each class is at most two runs: ncols[0] = all columns,
// ncols[1] = the shared wide columns, ncols[2] = the shared columns, ncols[3] = the end of the routed wide ones.
__global__ void __launch_bounds__(256) k_pf_cols(const int * __restrict__ act, const int * __restrict__ nact_p, const int * __restrict__ offsets,
                                                int n, int P, int4 * __restrict__ cols, int * __restrict__ ncols) {
    __shared__ int scw[256], scn[256];
    const int i = threadIdx.x, nact = *nact_p, nsh = (n + PF_TOK - 1) / PF_TOK;
    int e = 0, s0 = 0, cnt = 0;
    if (i < nact) { e = act[i]; s0 = offsets[e]; cnt = offsets[e + 1] - s0; }
    const int rem = cnt % PF_TOK, nw = cnt / PF_TOK + (rem > PF_TOK / 2 ? 1 : 0), nn = rem > 0 && rem <= PF_TOK / 2 ? 1 : 0;
    scw[i] = nw; scn[i] = nn;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {   // inclusive scans
        const int vw = i >= off ? scw[i - off] : 0, vn = i >= off ? scn[i - off] : 0;
        __syncthreads();
        scw[i] += vw; scn[i] += vn;
        __syncthreads();
    }
    const int tw = scw[255], bw = nsh + scw[i] - nw, bn = nsh + tw + scn[i] - nn;
    for (int c = 0; c < nw; ++c) { cols[bw + c] = make_int4(i, s0 + PF_TOK * c, min(PF_TOK, cnt - PF_TOK * c), e); }
    if (nn) { cols[bn] = make_int4(i, s0 + cnt - rem, rem, e); }
    for (int c = i; c < nsh; c += 256) { cols[c] = make_int4(-1, P + PF_TOK * c, min(PF_TOK, n - PF_TOK * c), 0); }
    if (i == 255) {
        const int rs = n % PF_TOK;
        ncols[0] = nsh + tw + scn[255]; ncols[1] = nsh - (rs > 0 && rs <= PF_TOK / 2 ? 1 : 0); ncols[2] = nsh; ncols[3] = nsh + tw;
    }
}
int prefill_shared_cols(int n) { return (n + PF_TOK - 1) / PF_TOK; }
hipError_t launch_prefill_cols(const int * act, const int * nact, const int * offsets, int n, int P, int4 * cols, int * ncols, hipStream_t st) {
    k_pf_cols<<<1, 256, 0, st>>>(act, nact, offsets, n, P, cols, ncols);
    return hipGetLastError();
}

// Q8_K integers as fp16 (exact): the MFMA operand copy of an activation array
__global__ void __launch_bounds__(256) k_q8_to_h(const int8_t * __restrict__ q, _Float16 * __restrict__ h, int64_t n) {
    const int64_t i = ((int64_t) blockIdx.x * 256 + threadIdx.x) * 8;
    if (i >= n) { return; }
    const u32x2 v = *(const LK_GLOBAL u32x2 *) (q + i);
    h8 o;
#pragma unroll
    for (int k = 0; k < 4; ++k) { o[k] = (_Float16) (int8_t) (v.x >> (8 * k)); o[4 + k] = (_Float16) (int8_t) (v.y >> (8 * k)); }
    *(LK_GLOBAL h8 *) (h + i) = o;
}
hipError_t launch_q8_to_h(const int8_t * q, _Float16 * h, int64_t n, hipStream_t st) {
    if (n <= 0) { return hipSuccess; }
    if (n % 8) { return hipErrorInvalidValue; }
    k_q8_to_h<<<(unsigned) ((n / 8 + 255) / 256), 256, 0, st>>>(q, h, n);
    return hipGetLastError();
}

// ---------------------------------------------------------------- the grouped GEMM
// NMAT = 2: gate/up (K = 7168, rows 2048, B rows = tokens, writes h); NMAT = 1: down (K = 2048, rows 7168, B rows =
// slots, writes o). Two kernels take the columns of launch_prefill_cols by class:
//   * wide (W = 8 waves, CPW = 2 16-row tiles per wave, columns of 33-64 slots, up to 4 token tiles): a wave's tiles
//     are the gate and up rows of one 16-row tile (gate/up: h forms in registers) or two row tiles (down);
//   * narrow (W = 16 waves, CPW = 1, columns of at most 32 slots, up to 2 token tiles): about half the registers per
//     wave, so four waves share a SIMD and hide more of the LDS read -> dequantise -> MFMA chain; gate/up hands g to
//     the up waves through LDS.
// Either way an item is (column, row group) and every output is computed once, in the same arithmetic.
template <int NMAT, int NB, int W, int CPW>
struct PfGeo {
    static constexpr bool NARROW = CPW == 1;
    static constexpr int NTM = NARROW ? 2 : PF_NTM;             // token tiles per column at most
    static constexpr int TPM = W * CPW / NMAT;                  // 16-row tiles per matrix in an item
    static constexpr int ROWS = TPM * 16, K = NB * QK, NTH = W * 64;
    static constexpr int BUF = NTM * PB_TILE;                   // one activation buffer
    static constexpr int L_G = L_PB + 2 * BUF;                  // narrow gate/up: g of the gate waves [8][64 lanes][2 tiles][4]
    static constexpr int LDS = L_G + (NARROW && NMAT == 2 ? 8 * 64 * NTM * 16 : 0);
    static_assert(LDS <= 160 * 1024 && W * CPW % NMAT == 0, "prefill GEMM geometry");
    // the matrix and the 16-row tile (within the item) of combo c of wave w
    __device__ static constexpr int mat(int w, int c) { return CPW == NMAT ? c : NMAT == 1 ? 0 : w / (W / NMAT); }
    __device__ static constexpr int tile(int w, int c) { return CPW == NMAT ? w : NMAT == 1 ? w * CPW + c : w % (W / NMAT); }
};

struct PfLane {
    int r, g;                 // row (token) in a 16-tile, chunk / lane group
    uint32_t trg, trs;        // table addresses with this lane's copy
};

// activation rows in LDS: see pf_swz (moe_common.h); lane (r, g)'s chunk 8 g + t sits at slot (8 pf_swz2(g) + t) ^ r
__device__ __forceinline__ int pf_swz2(int g) { return ((g & 1) << 1) | (g >> 1); }

// one block of one 16-row tile: the tiled chunk g of row r (qs) and d
struct PfW { u32x4 q; uint16_t d; };

// raw buffer resource over p (gfx9 word 3; the record count only bounds offsets, which stay far below it)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t pf_rsrc(const void * p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short) 0, 0x7fffffff, 0x00020000);
}
// a wave-uniform pointer kept in scalar registers
__device__ __forceinline__ const uint8_t * pf_uniform(const uint8_t * p) {
    const uint64_t v = (uint64_t) p;
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) (v >> 32));
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) v);
    return (const uint8_t *) (((uint64_t) hi << 32) | (uint64_t) lo);
}

// 16 bytes per lane from a buffer straight into LDS (lane L at dst + 16 L); the builtin exists for the device pass only,
// so the host pass (which instantiates the kernel's launch stub) sees an empty body
__device__ __forceinline__ void buf_lds16(__amdgpu_buffer_rsrc_t r, LK_LOCAL uint8_t * dst, uint32_t voff, uint32_t soff) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LK_LOCAL void *) dst, 16, voff, soff, 0, 0);
#else
    (void) r; (void) dst; (void) voff; (void) soff;
#endif
}
__device__ __forceinline__ void dma16(const void * src, LK_LOCAL uint8_t * dst) {
    __builtin_amdgcn_global_load_lds((const LK_GLOBAL void *) src, (LK_LOCAL void *) dst, 16, 0, 0);
}

// the columns of one class inside [col0, col1): two runs [a0, a1) and [b0, b1) of the column table (k_pf_cols' order)
struct PfRuns {
    int a0, na, b0, nb;
    __device__ int count() const { return na + nb; }
    __device__ int col(int j) const { return j < na ? a0 + j : b0 + (j - na); }
};
__device__ __forceinline__ int pf_clip(int lo, int hi, int c0, int c1, int & start) {
    start = lo > c0 ? lo : c0;
    const int end = hi < c1 ? hi : c1;
    return end > start ? end - start : 0;
}
template <bool NARROW>
__device__ __forceinline__ PfRuns pf_runs(const PrefillArgs & a) {
    const int total = gptr(a.ncols)[0], shw = gptr(a.ncols)[1], sh = gptr(a.ncols)[2], rw = gptr(a.ncols)[3];
    const int c0 = a.col0, c1 = a.col1 > 0 ? a.col1 : total;
    PfRuns r;
    if (NARROW) { r.na = pf_clip(shw, sh, c0, c1, r.a0); r.nb = pf_clip(rw, total, c0, c1, r.b0); }
    else { r.na = pf_clip(0, shw, c0, c1, r.a0); r.nb = pf_clip(sh, rw, c0, c1, r.b0); }
    return r;
}

template <int NMAT, int NB, int W, int CPW>
__global__ void __launch_bounds__(W * 64, 1) k_pf_gemm(const PrefillArgs a) {
#pragma clang fp contract(off)
    using Geo = PfGeo<NMAT, NB, W, CPW>;
    constexpr int C = CPW;
    extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds[];
    LK_LOCAL uint8_t * lds = (LK_LOCAL uint8_t *) dyn_lds;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = lane_id();
    if (lds_addr(dyn_lds) & 0xFFFFu) {   // table addressing needs a 64 KB aligned base
        if (threadIdx.x == 0) {
            __hip_atomic_fetch_or(gptr(a.err), 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (a.herr) { __hip_atomic_store(gptr(a.herr), 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM); }
        }
        return;
    }
    // tables into LDS (direct loads), visible after vmcnt(0) + the first barrier
    for (int c = wave; c < PTAB_BYTES / 1024; c += W) { dma16(a.ptab + c * 64 + lane, lds + c * 1024); }
    PfLane ln;
    ln.r = lane & 15; ln.g = lane >> 4;
    ln.trg = (uint32_t) L_PG | ((uint32_t) ln.r << 4);
    ln.trs = (uint32_t) L_PS | ((uint32_t) ln.r << 4);
    const PfRuns runs = pf_runs<Geo::NARROW>(a);
    const int nrg = a.R / Geo::ROWS;
    const size_t dreg = (size_t) (a.R / 64) * NB * 4096;   // d region offset of a tiled matrix
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();

    for (int it = blockIdx.x; it < runs.count() * nrg; it += gridDim.x) {
        const int col = runs.col(it / nrg), rg = it % nrg;
        const u32x4 cv = *(const LK_GLOBAL u32x4 *) (a.cols + col);
        const int4 cd = make_int4((int) cv.x, (int) cv.y, (int) cv.z, (int) cv.w);
        const bool routed = cd.x >= 0;
        const int sb = cd.y, sc = cd.z;
        // B rows of the copy instructions: instruction i copies rows 2 i and 2 i + 1 (lane half L >> 5)
        auto brow = [&](int n32) -> int {
            const int s = sb + (n32 < sc ? n32 : 0);
            return NMAT == 2 ? (routed ? gptr(a.perm)[s] / a.topk : s - a.P) : s;
        };
        // Buffer loads: a scalar resource (base, no bounds that matter) + a 32-bit lane offset + a scalar block offset,
        // so no 64-bit per-lane address lives in vector registers.
        const __amdgpu_buffer_rsrc_t rb = pf_rsrc(a.bh), rd = pf_rsrc(a.bd);
        const uint32_t oX = (uint32_t) brow(lane) * (NB * 4);   // lane n loads the scale of token n of the column
        // the wave's tiles: combo c = (matrix Geo::mat, 16-row tile Geo::tile): scalar resources at the tile's qs / d
        // bases, the lane's offset (chunk g of row r) in one vector register
        __amdgpu_buffer_rsrc_t uq[C], ud[C];
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const int mat = Geo::mat(wave, c), ti = Geo::tile(wave, c);
            const uint8_t * Wm = routed ? a.w[mat] + (size_t) cd.w * a.estride : a.sh[mat];
            const int row0 = rg * Geo::ROWS + ti * 16;   // a 16-row tile lies inside one 64-row group
            const int g64 = row0 >> 6, r0 = row0 & 63;
            uq[c] = pf_rsrc(pf_uniform(Wm + (size_t) g64 * NB * 4096 + r0 * 16));
            ud[c] = pf_rsrc(pf_uniform(Wm + dreg + (size_t) g64 * NB * 128 + r0 * 2));
        }
        const uint32_t lq = (uint32_t) ln.g * 1024 + (uint32_t) ln.r * 16, ldo = (uint32_t) ln.r * 2;
        auto load_w = [&](int j, PfW (&w)[C]) {
#pragma unroll
            for (int c = 0; c < C; ++c) {
                w[c].q = __builtin_amdgcn_raw_buffer_load_b128(uq[c], lq, j * 4096, 2);   // nt: streamed once
                w[c].d = __builtin_amdgcn_raw_buffer_load_b16(ud[c], ldo, j * 128, 0);
            }
        };
        auto run_item = [&](auto ntc) {
            constexpr int NT = decltype(ntc)::value;   // token tiles of the column (1, 2 or 4)
            // the column's activations of block j go straight from memory into LDS buffer j % 2 (buffer loads to LDS:
            // lane L's 16 bytes land at L * 16 of the instruction's 1 KB, no registers): copy instruction i covers token
            // rows 2 i + (lane / 32), i < 8 NT, taken by waves i % W; lane L < 32 of a row takes the row's chunk
            // pf_swz(L ^ (row % 16)) -- the swizzle applied on the memory side. Lane n also loads token n's block scale
            // into a register.
            constexpr int NI = (8 * NT + W - 1) / W;   // copy instructions per wave (some waves of the narrow kernel none)
            struct PfB { float dx; };
            uint32_t ob[NI];
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int row = 2 * (wave + W * i) + (lane >> 5);
                ob[i] = (uint32_t) brow(row < 16 * NT ? row : 0) * (Geo::K * 2) + pf_swz((uint32_t) ((lane & 31) ^ (row & 15))) * 16;
            }
            auto load_b = [&](int j, PfB & bq, int buf) {
                LK_LOCAL uint8_t * dst = lds + L_PB + buf * Geo::BUF;
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    if (wave + W * i < 8 * NT) { buf_lds16(rb, dst + 2 * (wave + W * i) * 512, ob[i], j * (QK * 2)); }
                }
                bq.dx = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rd, oX, j * 4, 0));
            };
            f4 acc[C][NT];
#pragma unroll
            for (int c = 0; c < C; ++c) { for (int tt = 0; tt < NT; ++tt) { acc[c][tt] = (f4) { 0.f, 0.f, 0.f, 0.f }; } }

            // one block: dequantise the C tiles step by step and run the MFMA chains of the token tiles
            auto block = [&](int j, const PfW (&w)[C], int buf, float dxl) {
                static_assert((L_PB % 512) == 0 && (Geo::BUF % 512) == 0, "XOR addressing inside 512-byte rows");
                const uint32_t bx = ((uint32_t) (L_PB + buf * Geo::BUF) + (uint32_t) ln.r * 512) | ((uint32_t) ((8 * pf_swz2(ln.g)) ^ ln.r) << 4);
                f4 cc[C][NT], cd[C][NT];   // the two exact chains: steps 0-3, steps 4-7
                h2v sc[C][2];
                uint32_t ms[C][2];
#pragma unroll
                for (int c = 0; c < C; ++c) {
                    const _Float16 s0 = (_Float16) iq2_scale(w[c].q.y), s1 = (_Float16) iq2_scale(w[c].q.w);
                    sc[c][0] = (h2v) { s0, s0 }; sc[c][1] = (h2v) { s1, s1 };
                    ms[c][0] = w[c].q.y & 0x7f7f7f7fu; ms[c][1] = w[c].q.w & 0x7f7f7f7fu;
                }
                // step t's LDS reads (the activation chunks, per tile a codebook and a sign entry) are issued one step
                // ahead of their use, into the other of two register sets
                struct Lk { u32x4 g[C], s[C]; h8 x[NT]; };
                auto lookup = [&](int t, Lk & k) {
                    const uint32_t bo = bx ^ ((uint32_t) t << 4);   // chunk (8 g + t) ^ r of the lane's token row
#pragma unroll
                    for (int tt = 0; tt < NT; ++tt) { k.x[tt] = __builtin_bit_cast(h8, *(const LK_LOCAL u32x4 *) (size_t) (bo + tt * PB_TILE)); }
#pragma unroll
                    for (int c = 0; c < C; ++c) {
                        const uint32_t a0 = t < 4 ? w[c].q.x : w[c].q.z, a1 = ms[c][t >> 2];
                        uint32_t ga, sa;
                        switch (t & 3) {
                        case 0: ga = tab_addr<0>(a0, ln.trg); sa = tab_addr<0>(a1, ln.trs); break;
                        case 1: ga = tab_addr<1>(a0, ln.trg); sa = tab_addr<1>(a1, ln.trs); break;
                        case 2: ga = tab_addr<2>(a0, ln.trg); sa = tab_addr<2>(a1, ln.trs); break;
                        default: ga = tab_addr<3>(a0, ln.trg); sa = tab_addr<3>(a1, ln.trs); break;
                        }
                        k.g[c] = *(const LK_LOCAL u32x4 *) (size_t) ga;
                        k.s[c] = *(const LK_LOCAL u32x4 *) (size_t) sa;
                    }
                };
                auto compute = [&](int t, const Lk & k) {
#pragma unroll
                    for (int c = 0; c < C; ++c) {
                        const h8 gs = __builtin_bit_cast(h8, k.g[c] ^ k.s[c]);
                        const h2v s = sc[c][t >> 2];
                        const h8 wv = gs * (h8) { s[0], s[1], s[0], s[1], s[0], s[1], s[0], s[1] };
                        const f4 z = (f4) { 0.f, 0.f, 0.f, 0.f };
#pragma unroll
                        for (int tt = 0; tt < NT; ++tt) {
                            if (t < 4) {
                                cc[c][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k.x[tt], wv, t == 0 ? z : cc[c][tt], 0, 0, 0);
                            } else {
                                cd[c][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k.x[tt], wv, t == 4 ? z : cd[c][tt], 0, 0, 0);
                            }
                        }
                    }
                };
                if constexpr (C * NT <= 4) {   // two register sets: step t + 1's reads issued before step t's MFMAs
                    Lk ka, kb;
                    lookup(0, ka);
#pragma unroll
                    for (int t = 0; t < 8; t += 2) {
                        lookup(t + 1, kb);
                        compute(t, ka);
                        if (t + 2 < 8) { lookup(t + 2, ka); }
                        compute(t + 1, kb);
                    }
                } else {                       // more tiles: one set (the step's MFMAs cover the next reads' latency)
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        Lk k; lookup(t, k); compute(t, k);
                        __builtin_amdgcn_sched_barrier(0);   // steps stay in order: reads of later steps are not hoisted
                    }
                }
                // block fold, in block order: y += (d_w * d_x) * bsum, bsum = the two chains' exact totals added once; the
                // scale of token 16 tt + 4 g + i comes from the lane that loaded it
                float dx[NT][4];
#pragma unroll
                for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        dx[tt][i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * (16 * tt + 4 * ln.g + i), __builtin_bit_cast(int, dxl)));
                    }
                }
#pragma unroll
                for (int c = 0; c < C; ++c) {
                    const float dw = h2f(w[c].d);
#pragma unroll
                    for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) { acc[c][tt][i] = acc[c][tt][i] + (dw * dx[tt][i]) * (cc[c][tt][i] + cd[c][tt][i]); }
                    }
                }
                (void) j; (void) buf;
            };

            // pipeline: weights two blocks ahead (three register stages), activations one block ahead (registers, then
            // the other of two LDS buffers). Every step issues the same loads (indices clamped at the last blocks: those
            // copies land in registers nobody reads any more), so the compiler's waits count them exactly.
            // short rows (down, 8 blocks) and items of many tiles keep the weights one block ahead (two stages): their
            // register budget is tighter
            constexpr int WA = (NB <= 8 || C * NT > 4 || Geo::NARROW) ? 1 : 2;   // narrow: four waves per SIMD hide it instead
            PfW w0[C], w1[C], w2[C];
            PfB bq;
            load_w(0, w0);
            if (WA == 2) { load_w(1, w1); }
            load_b(0, bq, 0);
            __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): block 0's activations are in LDS
            __syncthreads();
            auto step = [&](int j, PfW (&cur)[C], PfW (&ahead)[C]) {
                const float dxl = bq.dx;             // block j's scale (loaded with its activations)
                // buffer (j + 1) % 2 was last read in step j - 1, before its barrier
                load_b(j + 1 < NB ? j + 1 : NB - 1, bq, (j + 1) & 1);
                load_w(j + WA < NB ? j + WA : NB - 1, ahead);
                __builtin_amdgcn_sched_barrier(0);   // nothing of the block moves above the loads
                block(j, cur, j & 1, dxl);
                __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): block j + 1's activations have landed in LDS (and the
                __builtin_amdgcn_s_barrier();       // weights of the next block are in): the barrier publishes them
            };
            if constexpr (WA == 1) {   // step j uses stage j % 2 and refills the other with block j + 1
                static_assert(NB % 2 == 0, "two steps per trip");
#pragma unroll 1
                for (int j = 0; j < NB; j += 2) { step(j, w0, w1); step(j + 1, w1, w0); }
            } else {                   // step j uses stage j % 3 and refills the stage of block j - 1 with block j + 2
                constexpr int NB3 = NB - NB % 3;
                int j = 0;
#pragma unroll 1
                for (; j < NB3; j += 3) {
                    step(j, w0, w2);
                    step(j + 1, w1, w0);
                    step(j + 2, w2, w1);
                }
                if (NB % 3 >= 1) { step(j, w0, w2); }
                if (NB % 3 == 2) { step(j + 1, w1, w0); }
            }

            // outputs: lane (r, g) holds tokens 4 g + i of each token tile for row r of each of its tiles
            if constexpr (NMAT == 2 && C == 1) {
                // narrow gate/up: the gate waves (0..7) leave 0.125 g in LDS, the up waves (8..15) form h for the same
                // tile. The exchange area is last read in this item; the next item's first barrier orders its reuse.
                LK_LOCAL float * xg = reinterpret_cast<LK_LOCAL float *>(lds + Geo::L_G);
                const int ti = Geo::tile(wave, 0);
                if (Geo::mat(wave, 0) == 0) {
#pragma unroll
                    for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) { xg[((ti * 64 + lane) * Geo::NTM + tt) * 4 + i] = 0.125f * acc[0][tt][i]; }
                    }
                }
                __syncthreads();
                if (Geo::mat(wave, 0) == 1) {
                    const int row = rg * Geo::ROWS + ti * 16 + ln.r;
#pragma unroll
                    for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int n32 = 16 * tt + 4 * ln.g + i;
                            if (n32 < sc) {
                                const size_t o = (size_t) (sb + n32) * a.R + row;
                                const float gv = xg[((ti * 64 + lane) * Geo::NTM + tt) * 4 + i], uv = 0.125f * acc[0][tt][i];
                                a.out[o] = det_silu(gv) * uv;
                                if (a.gdbg) { a.gdbg[o] = gv; a.udbg[o] = uv; }
                            }
                        }
                    }
                }
            } else {
                constexpr int RT = NMAT == 2 ? 1 : C;   // row tiles of the wave (gate/up wide: one, both matrices)
#pragma unroll
                for (int c = 0; c < RT; ++c) {
                    const int row = rg * Geo::ROWS + Geo::tile(wave, c) * 16 + ln.r;
#pragma unroll
                    for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int n32 = 16 * tt + 4 * ln.g + i;
                            if (n32 < sc) {
                                const size_t o = (size_t) (sb + n32) * a.R + row;
                                if (NMAT == 2) {
                                    const float gv = 0.125f * acc[0][tt][i], uv = 0.125f * acc[1][tt][i];
                                    a.out[o] = det_silu(gv) * uv;
                                    if (a.gdbg) { a.gdbg[o] = gv; a.udbg[o] = uv; }
                                } else {
                                    a.out[o] = 0.125f * acc[c][tt][i];
                                }
                            }
                        }
                    }
                }
            }
        };
        if constexpr (Geo::NARROW) {
            if (sc > 16) { run_item(std::integral_constant<int, 2>{}); }
            else { run_item(std::integral_constant<int, 1>{}); }
        } else {
            run_item(std::integral_constant<int, 4>{});   // a wide column: 33..64 slots
        }
    }
}

template <int NMAT, int NB, int W, int CPW>
static hipError_t pf_setup() {
    return hipFuncSetAttribute((const void *) k_pf_gemm<NMAT, NB, W, CPW>, hipFuncAttributeMaxDynamicSharedMemorySize,
                               PfGeo<NMAT, NB, W, CPW>::LDS);
}
hipError_t prefill_init() {
    hipError_t e = pf_setup<2, 28, 8, 2>();
    if (e == hipSuccess) { e = pf_setup<1, 8, 8, 2>(); }
    if (e == hipSuccess) { e = pf_setup<2, 28, 16, 1>(); }
    if (e == hipSuccess) { e = pf_setup<1, 8, 16, 1>(); }
    return e;
}

// the wide kernel, then the narrow one, over the columns col0 .. col1 - 1 (each takes its class)
hipError_t launch_prefill_gemm(const PrefillArgs & a, int grid, hipStream_t st) {
    if (grid < 1 || !a.ptab || !a.cols || !a.ncols || !a.bh || !a.bd || !a.out || !a.err) { return hipErrorInvalidValue; }
    if (a.nmat == 2) {
        if (a.K != 28 * QK || a.R % PfGeo<2, 28, 8, 2>::ROWS || a.R % PfGeo<2, 28, 16, 1>::ROWS || !a.w[0] || !a.w[1] || !a.sh[0] || !a.sh[1] || !a.perm) {
            return hipErrorInvalidValue;
        }
        k_pf_gemm<2, 28, 8, 2><<<grid, 8 * 64, PfGeo<2, 28, 8, 2>::LDS, st>>>(a);
        k_pf_gemm<2, 28, 16, 1><<<grid, 16 * 64, PfGeo<2, 28, 16, 1>::LDS, st>>>(a);
    } else if (a.nmat == 1) {
        if (a.K != 8 * QK || a.R % PfGeo<1, 8, 8, 2>::ROWS || a.R % PfGeo<1, 8, 16, 1>::ROWS || !a.w[0] || !a.sh[0]) { return hipErrorInvalidValue; }
        k_pf_gemm<1, 8, 8, 2><<<grid, 8 * 64, PfGeo<1, 8, 8, 2>::LDS, st>>>(a);
        k_pf_gemm<1, 8, 16, 1><<<grid, 16 * 64, PfGeo<1, 8, 16, 1>::LDS, st>>>(a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace lk
