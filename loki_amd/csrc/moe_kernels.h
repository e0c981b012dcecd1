// moe_kernels.h -- host-side launchers of the MoE-block kernels (internal to libloki_moe; the C ABI is include/loki_moe.h).
// Every launcher enqueues on the given stream and returns hipGetLastError() of its launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace lk {

// Q8_K of nrows rows of K floats (K % 256 == 0): q [nrows][K], d [nrows][K/256]
hipError_t launch_quant_q8k(const float * x, int64_t nrows, int K, int8_t * q, float * d, hipStream_t st);

// router logits [n][n_exp] under the fp64 chunk contract (K % 256 == 0)
// part2: fp64 scratch of router_split_doubles(n, n_exp, K) for the K-split tiles (RL_SPLIT_MIN <= n <= RL_SPLIT_MAX,
// K 7168); may be null (then the split is not used)
constexpr int RL_SPLIT_MIN = 40;     // below it one workgroup per expert (k_router_wg) is as fast or faster
constexpr int RL_SPLIT_MAX = 2048;   // above it the whole LDS tiles (scratch 16 x n x n_exp doubles at most 64 MiB)
size_t router_split_doubles(int n, int n_exp, int K);
hipError_t launch_router_logits(const float * W, const float * x, int n, int n_exp, int K, float * logits, double * part2, hipStream_t st);
// sigmoid, bias, grouped top-k, normalised weights; probs [n][n_exp], sel/wts [n][keep]: with 0 < keep < topk each
// row keeps its keep heaviest picks (rescaled to sum to renorm when renorm > 0), else all topk
hipError_t launch_router_select(const float * logits, const float * bias, int n, int n_exp, int n_group, int topk_group,
                                int topk, float scale, float * probs, int * sel, float * wts, hipStream_t st, int keep = 0,
                                float renorm = 0.f);

// the engine's --share-experts keep (src/server_core_fused.cpp:798-806) of n rows' topk picks sel8 / w8 [n][topk] (pick
// order, n_exp <= 256) into sel / wts [n][ke] in kept order, rescaled to renorm when renorm > 0
hipError_t launch_keep_share(const int * sel8, const float * w8, int n, int topk, int ke, float renorm, int * sel, float * wts, hipStream_t st);

// both in one launch for n <= 8 tokens and K = 7168 (router_fused_ok): the last workgroup to finish its logits selects,
// reading the others' logits as epoch-tagged words tl [n][n_exp] (zero or older epochs before the launch). cnt: a
// device word that is zero before the launch and left zero; done (may be null): host memory set to epoch once sel and
// wts are written (system scope); err / herr (may be null): device and mapped host words that get code 2 if a poll of
// the tagged logits times out (the picks are then -1)
bool router_fused_ok(int n, int K);
hipError_t launch_router_fused(const float * W, const float * x, int n, int n_exp, int K, float * logits, const float * bias, int n_group,
                               int topk_group, int topk, float scale, float * probs, int * sel, float * wts, uint64_t * tl,
                               unsigned epoch, unsigned * cnt, unsigned * done, int * err, int * herr, hipStream_t st, int keep = 0,
                               float renorm = 0.f);

// stable counting sort of the P = n*topk pairs by expert: counts [n_exp], offsets [n_exp+1], perm/inv [P],
// act = used experts ascending, nact = their number (device scalar)
// scratch (may be null: one workgroup for every size): dispatch_scratch_ints(P) ints, used above 4096 pairs
size_t dispatch_scratch_ints(int P);
hipError_t launch_dispatch(const int * sel, int P, int n_exp, int * counts, int * offsets, int * perm, int * inv,
                           int * act, int * nact, hipStream_t st, int * scratch = nullptr);

struct ExpertArgs {
    const uint4 * tab;               // LDS table image (build_table_image)
    const uint8_t * w[2];            // routed expert bases (tiled layout) of matrix 0 / 1, expert e at w + e * estride
    size_t estride;
    const uint8_t * sh[2];           // shared expert matrices (tiled)
    const int8_t * aq; const float * ad;   // Q8_K activations (K columns): gate/up rows = tokens, down rows = slots
    int K, R, nmat;                  // columns, rows per matrix, matrices per task set (2 = gate+up, 1 = down)
    const int * act, * nact, * offsets, * perm;
    int topk, n, P, shared;          // shared: 1 = the shared expert runs as slot m == nact (tokens 0..n-1, slots P..)
    float * terms;                   // unused (no block-term scratch)
    unsigned * cnt_rg, * cnt_2, * queue;   // self-resetting counters (zero before the first launch); queue unused
    float * h; int8_t * hq; float * hd;    // gate/up epilogue: h [P+n][R] and its Q8_K
    float * gdbg, * udbg;                  // optional gate / up outputs
    float * o;                             // down epilogue: o [P+n][R]
    const int * inv; const float * wts; float * y;   // down: fused k-ordered combine when y != null
};
// persistent launches: grid = workgroups (one per CU); experts_init sets the LDS limit once per process
hipError_t experts_init();
size_t experts_terms_floats(int nmat, int slots, int R, int K);
// the image of the codebook / sign-mask LDS tables (TAB_BYTES, 96 KB), built once per context
hipError_t build_table_image(uint4 * img, hipStream_t st);
hipError_t launch_experts_gateup(const ExpertArgs & a, int grid, hipStream_t st);
hipError_t launch_experts_down(const ExpertArgs & a, int grid, hipStream_t st);

// ---------------------------------------------------------------- single-launch decode block (moe_decode.hip)
struct DecodeArgs {
    const uint4 * tab;
    const float * x; int n;                          // tokens [n][E], n <= 8
    int prenorm; const float * nw; float eps;        // prenorm: the block's input is RMSNorm(x) * nw (nw null: ones)
    const float * resid;                             // added to the block's output when not null ([n][E])
    const float * Wr; const float * bias; int n_exp, n_group, topk_group, topk; float scale;
    int keep; float renorm;                          // experts kept per token (keep <= topk; the slots use keep), rescale
    const uint8_t * gate, * up, * down; size_t estride;   // routed experts (tiled), expert e at + e * estride
    const uint8_t * sh_gate, * sh_up, * sh_down;
    // 0: every matrix IQ2_XXS (tiled). KF_Q2K / KF_Q3K (kquant_device.h; the one-token kernel only): the routed down
    // in that K-quant and the shared expert in Q5_K / Q5_K / Q6_K, ggml's block layout read in place, routed down
    // expert e at down + e * dstride
    int kdown; size_t dstride;
    // the one-token kernel only: the caller's picks (8 expert ids and weights on the device; null: the kernel routes).
    // Then the router and the selection are skipped and the combine is the reference fl_moe's (distinct ids ascending,
    // their weights summed in k order): moe_out = that sum, y = (moe_out + shared) + resid
    // (o_out, may be null: the 8 slots' outputs [slot][E], for the reference's per-slot attribution)
    const int * ext_sel; const float * ext_w; float * moe_out; float * o_out;
    int share;                                       // keep < topk by the engine's --share-experts rule (n <= 8 block)
    // the one-token kernel only. spec_combine: the kernel routes, then combines as fl_moe does on those picks (the
    // ext_sel combine; moe_out and resid required), and XCD 0's selecting wave writes the picks and weights to hsel
    // (8 ids, then 8 weights) and then *hdone = epoch (host-mapped, for fl_fetch). fdone (either path, may be null):
    // *fdone = epoch once every workgroup's outputs are written (fcnt: a device counter, zero before the launch,
    // reset by the last workgroup), so the host can wait on a word instead of the stream
    int spec_combine; int * hsel; unsigned * hdone; unsigned * fcnt, * fdone;
    // the one-token kernel, with fdone: tstamp [0] = workgroup 0's entry, [1] = the last workgroup's end (the 100 MHz
    // s_memrealtime clock; may be null), the launch's GPU time without events around it
    uint64_t * tstamp;
    int E, H;                                        // 7168, 2048 (the kernel's geometry)
    int8_t * xq; float * xd;                         // Q8_K of x (written by workgroup 0)
    float * logits, * probs; int * sel; float * wts; int * counts, * offsets, * perm, * inv, * act, * nact;
    // epoch-tagged words {epoch << 32 | 32-bit payload}: probabilities [n][n_exp], h [P+n][H] and o [P+n][E] per
    // dispatch slot
    uint64_t * tlogits, * th, * to;
    // the n <= 8 block's XCD-shared Q8_K of the tokens (null: every workgroup quantises all of them): per XCD a copy
    // of the staged token rows plus one epoch-tagged word per block (decode_xq_bytes() in all); only for a grid of 256
    // workgroups placed round-robin over the 8 XCDs (decode1_init's probe)
    uint8_t * xqx;
    float * y;                                       // [n][E]
    unsigned epoch; int * err;
    int * herr;                                      // host-mapped copy of a reported error code (may be null): the
                                                     // host sees a failed launch without synchronising
};
// sizes (64-bit words) of the tagged buffers for any n <= 8 (topk <= MAXK)
constexpr size_t DEC_TLOGITS = 8 * 256, DEC_TH = (size_t) 8 * (MAXK + 1) * 2048,
                 DEC_TO = (size_t) 8 * (MAXK + 1) * 7168;
hipError_t decode_init(int ncu, int * grid);
// routing rules the decode block supports (its selection keeps the group scores in registers)
bool decode_rule_ok(int n_exp, int n_group);
size_t decode_lds_bytes();
size_t decode_xq_bytes();
// grid workgroups (at most one per CU can be resident): a cooperative launch guarantees they are all resident; a
// regular launch assumes it (nothing else running on the CUs) -- a violation ends in a reported wait timeout
hipError_t launch_moe_decode(const DecodeArgs & a, int grid, bool cooperative, hipStream_t st);
// one decode token with all topk = 8 picks kept, organised by XCD (moe_decode1.hip): 256 workgroups, one per CU of a
// 256-CU device (*ok = 0 on other devices); same arguments, tagged buffers and results as launch_moe_decode
hipError_t decode1_init(int ncu, int * ok);
size_t decode1_lds_bytes();
hipError_t launch_moe_decode1(const DecodeArgs & a, bool cooperative, hipStream_t st);

// ---------------------------------------------------------------- prefill grouped GEMM on MFMA (moe_prefill.hip)
struct PrefillArgs {
    const uint4 * ptab;                  // fp16 table image (build_prefill_tables)
    const uint8_t * w[2]; size_t estride;   // routed matrices (tiled), expert e at + e * estride
    const uint8_t * sh[2];               // shared expert matrices (tiled)
    const int * perm; int topk, P;       // gate/up: slot -> token = perm[slot] / topk (shared slots P + t -> t)
    int R, K, nmat;                      // rows, columns; nmat 2 = gate/up, 1 = down
    const int4 * cols; const int * ncols;   // launch_prefill_cols
    const _Float16 * bh; const float * bd;  // activations: Q8_K integers as fp16 [rows][K] and scales [rows][K/256]
    float * out;                         // gate/up: h [P+n][R] (silu(g) * u); down: o [P+n][R]
    float * gdbg, * udbg;                // optional gate / up outputs
    int * err;                           // bit 4: the LDS base is not 64 KB aligned
    int * herr;                          // host-mapped copy of the code (may be null)
    // the columns col0 .. col1 - 1 of launch_prefill_cols (col1 <= 0: to the last); the shared expert's come first,
    // ceil(n / 64) of them
    int col0, col1;
    // launch_kq_gemm only: activation row = slot - arow0, output row = slot - orow0 (the shared expert's gate / up
    // read the tokens' rows and write rows 0 .. n - 1 of their own outputs)
    int arow0, orow0;
};
hipError_t prefill_init();
size_t prefill_table_bytes();
hipError_t build_prefill_tables(uint4 * img, hipStream_t st);
// columns of <= 64 slots (PF_TOK) of one expert: the shared expert's ceil(n / 64) first, then act order; cols sized
// >= prefill_shared_cols(n) + P / 64 + NEXP_MAX + 2
constexpr int PF_NCOLS = 4;   // the counts launch_prefill_cols writes (ncols[0] = all columns; the class boundaries)
hipError_t launch_prefill_cols(const int * act, const int * nact, const int * offsets, int n, int P, int4 * cols, int * ncols, hipStream_t st);
int prefill_shared_cols(int n);   // the shared expert's columns (the first ones) for n tokens
hipError_t launch_q8_to_h(const int8_t * q, _Float16 * h, int64_t n, hipStream_t st);
hipError_t launch_prefill_gemm(const PrefillArgs & a, int grid, hipStream_t st);

// K-quant matrices on the matrix cores (kq_gemm.hip), bit-identical to launch_kq_matvec: columns col0 .. col1 - 1 of
// launch_prefill_cols (routed: expert e at w[0] + e * estride; the shared expert's: sh[0]), ggml's blocks read in
// place; activations bh / bd = Q8_K integers as fp16 [rows][K] and their scales (row = slot - arow0), outputs
// out[(slot - orow0) * R + r]. fmt KF_Q2K / KF_Q3K / KF_Q6K with K = 2048 (downs), KF_Q5K with K = 7168 (the shared
// gate / up); R % 128 == 0.
hipError_t kq_gemm_init();
hipError_t launch_kq_gemm(const PrefillArgs & a, int fmt, int grid, hipStream_t st);

// y[t] = sum_k (o[inv[t*topk+k]] * w[t][k]) in k order + o[P+t] (+ resid[t] when given)
// grid y extent of the row-looping kernels: min(rows, cap); the cap is 65535 unless a test lowers it
void set_grid_ycap(int cap);
unsigned grid_y(int rows);
hipError_t launch_combine(const float * o, const int * inv, const float * wts, int n, int topk, int E, int P,
                          const float * resid, float * y, float * moe, hipStream_t st);

// ggml-layout IQ2_XXS matrices -> tiled layout (nmat matrices of R x K at the given byte strides)
hipError_t launch_pack_tiled(const uint8_t * src, size_t src_stride, uint8_t * dst, size_t dst_stride, int R, int K, int nmat, hipStream_t st);
hipError_t launch_unpack_tiled(const uint8_t * src, size_t src_stride, uint8_t * dst, size_t dst_stride, int R, int K, int nmat, hipStream_t st);

// synthetic data: IQ2_XXS matrices (qs uniform bytes, d = fp16(|N(0, sigma^2)|)) keyed by (seed, matrix id, row, block)
hipError_t launch_synth_iq2(uint8_t * dst, size_t dst_stride, int R, int K, int nmat, int layout, uint64_t seed,
                            uint64_t mat0, float sigma, hipStream_t st);
hipError_t launch_synth_normal(float * dst, int64_t count, uint64_t seed, uint64_t stream, float mean, float sigma, hipStream_t st);
// fp16 bits -> fp32 (exact widening)
hipError_t launch_f16_to_f32(const uint16_t * src, float * dst, int64_t count, hipStream_t st);

// ---------------------------------------------------------------- K-quant mat-vecs (kquant.hip)
struct KqArgs {
    const uint8_t * w; size_t estride;   // ggml-layout matrices [R][K/256 blocks], expert e at w + e * estride
    const int8_t * aq; const float * ad; // Q8_K activation rows [.][K], [.][K/256]: slot s reads row s
    int K, R;
    const int * act, * nact, * offsets; // act != null: workgroup row y = active expert act[y] (y < *nact), slots
                                         // offsets[e] .. offsets[e+1]; act == null: one matrix, slots 0 .. n-1
    int n;
    float * out; int ldo;                // out[s * ldo + r]
    int rw;                              // rows per workgroup tile (set by launch_kq_matvec)
    const uint8_t * w2; float * out2;    // act == null: a second matrix of the same shape and format on the same rows
                                         // (workgroup row y = 1), e.g. the shared expert's up beside its gate
};
// block bytes of a K-quant format code (FL_Q2K 84, FL_Q3K 110, FL_Q5K 176, FL_Q6K 210; 0 = not a K-quant)
int kq_block_bytes(int fmt);
// max_slots sizes the token groups (a bound or the expected slots of one expert; more run as extra groups);
// grid_experts >= *nact
hipError_t launch_kq_matvec(const KqArgs & a, int fmt, int max_slots, int grid_experts, hipStream_t st);
// h = silu(g) * u, element-wise under the exp contract
hipError_t launch_swiglu(const float * g, const float * u, int64_t n, float * h, hipStream_t st);
// the same h for nrows rows of K (K % 256 == 0) and its Q8_K (q [nrows][K], d [nrows][K/256]) in one pass
hipError_t launch_swiglu_q8k(const float * g, const float * u, int64_t nrows, int K, float * h, int8_t * q, float * d, hipStream_t st);

// ggml rms_norm (fp64 sum of fp32 squares) then the weight (w may be null = ones); one block per row
hipError_t launch_rmsnorm(const float * x, const float * w, float * y, int n, int D, float eps, hipStream_t st);

// element-wise probes of the exp contract (tests)
hipError_t launch_expf_probe(const float * x, float * y, int64_t n, int which, hipStream_t st);

}  // namespace lk
