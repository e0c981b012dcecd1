/* loki_moe.h -- C ABI of libloki_moe.so, the MI355X (gfx950) DeepSeek-R1 MoE feed-forward block.
 *
 * Drop-in for the MoE part of the reference's src/fused_layer.h: the same FLCtx / FLW / FLOut types and fl_* names and
 * parameter lists, with hipEvent_t where the reference has cudaEvent_t. Entry points marked "additive" have no
 * counterpart in the reference; they are the device-resident path (router, dispatch and experts on the GPU, no host
 * round-trip) that the MI355X build is measured on.
 *
 * Errors: the reference prints "[fused] CUDA error" and exits (src/fused_layer.cu:17). The reference-named entry points
 * keep that behaviour for runtime failures; the additive ones return 0 or a negative FL_E* code and leave a message in
 * fl_last_error(ctx) instead, so a host harness can test its error paths.
 * Threading: one HIP stream per context, not thread-safe (as the reference, src/fused_layer.cu:392-393).
 */
#pragma once
#include <stdint.h>
#include <stddef.h>
#include <hip/hip_runtime.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct FLCtx FLCtx;

/* formats (src/fused_layer.h:11): experts in FL_IQ2; routed down also FL_Q2K / FL_Q3K and the shared expert also
 * K-quants (the reference's real shards), read in place in ggml's block layout */
enum { FL_Q4K = 0, FL_Q6K = 1, FL_Q80 = 2, FL_Q5K = 3, FL_IQ2 = 4, FL_Q2K = 5, FL_Q3K = 6 };
/* IQ2_XXS byte layouts of expert matrices: ggml's row-major blocks, or the tiled resident layout of fl_pack_iq2xxs */
enum { FL_LAYOUT_GGML = 0, FL_LAYOUT_TILED = 1 };
/* status codes of the additive entry points */
enum { FL_OK = 0, FL_EINVAL = -1, FL_ENOMEM = -2, FL_EHIP = -3, FL_ERANGE = -4, FL_ESCOPE = -5 };

typedef struct FLW {   /* src/fused_layer.h:12-18, unchanged: device pointers of one layer's always-used weights */
    const void * attn_norm, * q_a, * q_a_norm, * q_b, * kv_a, * kv_a_norm, * kv_b, * k_bT, * attn_out, * ffn_norm, * gate_inp, * probs_b;
    const void * sh_gate, * sh_up, * sh_down;
    const void * d_gate, * d_up, * d_down;
    int kv_b_v;
    int gate_f16;
} FLW;

typedef struct FLOut {   /* src/fused_layer.h:19-21, unchanged: context-owned pinned host mirrors */
    const int * sel; const float * wts; const float * ncur; const float * fi; const float * skt; const int * sel_s; const float * wts_s;
    const float * sc; const float * ccat; const float * h; const float * moe;
} FLOut;

/* ---------------------------------------------------------------- reference entry points (src/fused_layer.h:22-53) */
/* fl.h:23 -- context: stream, events, buffers. kvp / sc_cap size the attention cache in the reference; kept for the ABI. */
FLCtx * fl_init(int kvp, int sc_cap);
/* fl.h:27 -- attention is outside this library: prints the reason and exits 7 like any fused-layer failure */
void fl_attn(FLCtx *, const FLW *, int N, int pos0, const int * pos, void * KC, void * VC, const float * hin, int dense, int last_row, int wrow);
/* fl.h:29 -- wide-pass buffers for wmax rows with KE experts per row */
int fl_wide_init(FLCtx *, int wmax, int KE);
/* fl.h:30 -- routed experts of one arena batch for up to 8 (row, k) pairs per slot; gate/up IQ2_XXS, down_fmt FL_Q2K,
 * FL_Q3K (the reference's, src/fused_layer.cu:541-550) or FL_IQ2; other codes exit 7 (the reference maps them to Q2_K) */
void fl_wide_moe(FLCtx *, const void * gate, const void * up, const void * down, int down_fmt, int nexp, const int * midx, const int * rows,
                 const int * kidx, const float * wk, int nslots, int KE, int par);
void fl_wide_mark(FLCtx *, int par);                 /* fl.h:31 */
void fl_wide_wait(FLCtx *, int par);                 /* fl.h:32 */
void fl_wide_finish(FLCtx *, int n, int KE, FLOut * out);   /* fl.h:33 -- h = base + sum_k out, moe = sum_k out, waited */
void fl_moe_outs(FLCtx *, int b, const int * ids, const float * w, int KE, float * out);   /* fl.h:35 */
void fl_wide_outs(FLCtx *, int row, int KE, float * out);                                  /* fl.h:36 */
void fl_wide_skip(FLCtx *, const float * mo, int n, FLOut * out);                         /* fl.h:37 */
/* fl.h:39 / fl.h:41 -- speculative attention and geometry sketch: outside this library (exit 7, as fl_attn) */
void fl_spec(FLCtx *, const FLW * W1, void * KC1, void * VC1);
void fl_sketch(FLCtx *, const float * TPROJ, const void * GSKT, int K);
/* fl.h:43 -- what & 1: sel/wts/ncur/fi of the last routing (fl_ffn_begin) to the host mirrors, waited; other bits are attention's */
void fl_fetch(FLCtx *, int n, int what, FLOut * out);
/* fl.h:45 -- narrow MoE (n <= 8): gate/up/down = arena bases of nexp experts in ggml layout at ggml stride (gate/up
 * IQ2_XXS; down in down_fmt = FL_Q2K or FL_Q3K as the reference, src/fused_layer.cu:599-608, or FL_IQ2), ids/w [n][KE]
 * with ids = slot indices into the arena; -> out->h = routed + shared + ffn_inp, out->moe = routed. Waited. */
void fl_moe(FLCtx *, const void * gate, const void * up, const void * down, int nexp, int down_fmt, const int * ids, const float * w, int KE, int n, FLOut * out);
void fl_skip(FLCtx *, const float * mo, int n, FLOut * out);                /* fl.h:47 -- h = mo + shared + ffn_inp, waited */
/* fl.h:49 -- host -> device on the context's stream, enqueued: a kernel reading the mapped memory when src is pinned
 * (hipHostMalloc'd; no copy engine, as src/fused_layer.cu:414-420), the copy engine when HIP cannot map src */
void fl_h2d(FLCtx *, void * dst, const void * src, size_t bytes);
void fl_wait_event(FLCtx *, hipEvent_t ev);                                 /* fl.h:51 */
double fl_gpu_ms(FLCtx *, int which);                                       /* fl.h:52 -- 1 = experts (ms, accumulated) */

/* additive: fl_h2d's bytes so far by kernel (mapped pinned) and by copy engine (the reference keeps the same two
 * counts and prints them once past 64 MB, src/fused_layer.cu:418-419) */
int fl_h2d_bytes(FLCtx *, size_t * by_kernel, size_t * by_copy_engine);

/* ---------------------------------------------------------------- additive: the MoE tail of fl_attn without attention
 * Router + shared expert on N rows (N <= 64 per call; wrow >= 0 places them at rows wrow.. of a wide pass), given the
 * ffn-normed rows ncur and the residual ffn_inp as host floats [N][7168] (the reference computes both inside fl_attn,
 * src/fused_layer.cu:498-525). Uses W->gate_inp (F32 [256][7168], or F16 with W->gate_f16), W->probs_b,
 * W->sh_gate/up/down (ggml layout, formats of fl_set_shared_formats).
 * One row after an fl_moe that ran on the routing's own picks over an arena declared with fl_register_tiled (a resident
 * arena, ids = expert ids): this call also runs that fl_moe's block on its own picks in the same launch as the routing
 * (speculatively; its outputs are used only by an fl_moe with exactly those ids, weights and arena pointers, which then
 * just waits for it -- FLDebug.kernel 3 -- and any other call runs as usual). The row and its residual go in by a small
 * copy kernel reading the pinned staging (no copy engine). Its time counts as fl_gpu_ms(1). */
int fl_ffn_begin(FLCtx *, const FLW * W, int N, const float * ncur, const float * ffn_inp, int wrow);
/* formats of W->sh_gate / sh_up / sh_down for fl_ffn_begin: FL_IQ2 (default, the all-IQ2_XXS configs) or K-quants;
 * the reference's shards are (FL_Q5K, FL_Q5K, FL_Q6K) (src/fused_layer.h:14; FLW carries no format). gate and up are
 * both FL_IQ2 or both K-quants. K-quant matrices are read in place and must be 4-byte aligned. */
int fl_set_shared_formats(FLCtx *, int gate_fmt, int up_fmt, int down_fmt);
/* routed experts behind fl_ffn_begin / fl_moe (default 256, the model's count; FLW carries no count) */
int fl_set_experts(FLCtx *, int n_exp);
/* routing rule: DeepSeek-V3 groups (default 8 groups, top-4 groups, top-8, x2.5); n_group = topk_group = 1 is the reference's rule */
int fl_set_routing(FLCtx *, int n_group, int topk_group, int topk, float scale);
/* keep-KE for fl_moe_layer / fl_moe_layer_normed (additive; the reference does it on the host between fl_fetch and
 * fl_moe, src/server_core_fused.cpp:793-813, with KE = 2 in production, :340): each row keeps its `keep` heaviest
 * routed experts (weight descending, equal weights in pick order) and, with renorm > 0, every kept weight is multiplied
 * by renorm / (their fp32 sum in kept order) when that sum exceeds 1e-6 (the reference: renorm 2.5, RENORM_EXPERTS on).
 * The block then runs keep slots per row; FLDebug's sel / wts hold [n][keep]. keep = 0 (default) keeps all topk.
 * fl_route_dev and fl_ffn_begin are unaffected (the engine's host dispatch applies its own keep). */
int fl_set_keep(FLCtx *, int keep, float renorm);
/* the engine's --share-experts rule for that keep (src/server_core_fused.cpp:798-806, flag at :376; loki/chat.py:35
 * runs the engine with --experts 3 --share-experts): with on != 0, keep < topk and n > 1 rows, every row keeps its own
 * min(2, keep) heaviest experts, then prefers its other picks (weight order) whose expert is among the rows' own, then
 * the rest in weight order, each such expert joining that set for the rows after it (rows in order). The kept list is
 * in that pick order, renormalised in that order. Default off. */
int fl_set_share_experts(FLCtx *, int on);

/* ---------------------------------------------------------------- additive: device-resident block (the measured path) */
typedef struct FLMoeLayer {
    const float * gate_inp;    /* [n_exp][E] F32 router weight (ffn_gate_inp), device */
    const float * probs_b;     /* [n_exp] F32 e_score_correction_bias (exp_probs_b), device */
    const void * gate_exps;    /* [n_exp] x IQ2_XXS [H rows][E cols] at expert stride H*E/256*66 B, device */
    const void * up_exps;      /* as gate_exps */
    const void * down_exps;    /* [n_exp] x IQ2_XXS [E rows][H cols] */
    const void * sh_gate, * sh_up, * sh_down;   /* shared expert, IQ2_XXS, same layout */
    int layout;                /* FL_LAYOUT_TILED (fl_pack_iq2xxs) */
    int n_exp;                 /* routed experts (<= 256) */
    int E, H;                  /* hidden (7168) and expert intermediate (2048) sizes; E, H multiples of 1024 */
} FLMoeLayer;
/* formats of fl_moe_layer's routed down and shared gate / up / down (default FL_IQ2 x 4; FLMoeLayer carries none):
 * FL_IQ2 matrices in the tiled layout, K-quants (the real shards' Q2_K / Q3_K down, Q5_K / Q5_K / Q6_K shared) read in
 * place in ggml's layout, 4-byte aligned. With any K-quant the block runs its per-pass kernels for every n. */
int fl_set_layer_formats(FLCtx *, int down_fmt, int sh_gate_fmt, int sh_up_fmt, int sh_down_fmt);
/* y[n][E] = MoE(x[n][E]) on the context's stream (x, y device pointers; asynchronous). n <= 65536.
 * Allocation extents are checked against the shapes (hipMemGetAddressRange) before any launch. */
int fl_moe_layer(FLCtx *, const FLMoeLayer * L, const float * x, int n, float * y);
/* the same on RMSNorm(h) * ffn_norm (ggml rms_norm with eps, then the norm weight; ffn_norm may be NULL: ones): the
 * layer's ffn_norm applied inside the block, as the reference's fl_attn applies it before the router (fl.cu:498). For
 * decode batches the norm runs inside the single launch; bit-identical to fl_rmsnorm_dev followed by fl_moe_layer.
 * residual != 0 adds h to the output (y = (moe + shared) + h, the reference combine's lo2 = moe + shared + fi,
 * fl.cu:366-372); h and y must then not alias. */
int fl_moe_layer_normed(FLCtx *, const FLMoeLayer * L, const float * ffn_norm, float eps, const float * h, int n,
                        int residual, float * y);
/* fl_moe_layer for one decode batch (1 <= n <= 8) that allocates no device memory. No counterpart in the reference: it
 * is for callers that cannot allocate -- code under HIP graph capture, serving loops that forbid hipMalloc. Same
 * arguments and result as fl_moe_layer (bit-identical y), under the context's routing rule, fl_set_keep and
 * fl_set_share_experts. It runs the single-launch decode block (tiled IQ2_XXS, E 7168, H 2048, a routing rule the
 * decode block takes: FL_ESCOPE otherwise) on a file-scope device array of 5,502,720 bytes that each GPU the library
 * runs on holds until the process ends (routing outputs, epoch-tagged hand-off words, the table image, an error word),
 * resolved and prepared per device by fl_init; it calls no hipMalloc / hipFree. Each call enqueues a fill kernel that
 * clears the hand-off words (never a memset) and the decode block, which tags them with one fixed epoch; it changes no
 * host-side state, so a call captured into a HIP graph is correct on every replay (set the context's stream to the
 * capture stream first). n above 8 is rejected with FL_ERANGE. Every call on one GPU shares that GPU's array, which
 * keeps the last call's contents: calls that overlap on one GPU (two streams, two contexts, two threads, two graphs)
 * race and give wrong results. Device-side failures are reported through fl_sync on the context that made the call.
 * FLDebug does not see this path's buffers. */
int fl_moe_layer_noalloc(FLCtx *, const FLMoeLayer * L, const float * x, int n, float * y);
/* router only: sel/w [n][topk] (device), logits/probs [n][n_exp] may be NULL */
int fl_route_dev(FLCtx *, const float * gate_inp, const float * probs_b, const float * x, int n, int n_exp, int E,
                 float * logits, float * probs, int * sel, float * w);
/* dispatch only: counts [n_exp], offsets [n_exp+1], perm/inv [n*topk], act [n_exp], nact [1] (device) */
int fl_dispatch_dev(FLCtx *, const int * sel, int n, int topk, int n_exp, int * counts, int * offsets, int * perm, int * inv, int * act, int * nact);
/* Q8_K of nrows x K floats (device): q [nrows][K] int8, d [nrows][K/256] */
int fl_quant_q8k_dev(FLCtx *, const float * x, int nrows, int K, int8_t * q, float * d);
/* y [n][R] = W . x_t for a K-quant matrix W (fmt FL_Q2K, FL_Q3K, FL_Q5K or FL_Q6K; R rows of K/256 ggml blocks, in
 * place, start and size multiples of 4 bytes) and n Q8_K rows q [n][K], d [n][K/256] (device; K % 256 == 0, K <= 8192).
 * The per-format mat-vec behind fl_moe / fl_ffn_begin (the reference's tc_matvec<F>, src/fused_layer.cu:102-158,
 * 203-254): integer sub-block sums exact, fp32 over the blocks in order (Q2_K bit-identical to ggml's scalar dot). */
int fl_kq_matvec_dev(FLCtx *, int fmt, const void * w, int R, int K, const int8_t * q, const float * d, int n, float * y);
/* IQ2_XXS ggml layout <-> tiled layout for nmat matrices of R x K at byte strides (device, may not alias) */
int fl_pack_iq2xxs(FLCtx *, const void * src_ggml, size_t src_stride, void * dst_tiled, size_t dst_stride, int R, int K, int nmat);
int fl_unpack_iq2xxs(FLCtx *, const void * src_tiled, size_t src_stride, void * dst_ggml, size_t dst_stride, int R, int K, int nmat);
/* Declares [base, base + bytes) (device) to hold IQ2_XXS matrices in the tiled layout (fl_pack_iq2xxs's output, or
 * fl_synth_iq2xxs with FL_LAYOUT_TILED); process-wide. fl_moe, fl_wide_moe and fl_ffn_begin read an arena or shared
 * matrix that lies wholly inside a declared range as it is, instead of repacking it from ggml's layout on every call
 * (the reference refills its arenas in place, src/server_core_fused.cpp:295-305, so memory not declared is always
 * repacked). A resident 256-expert arena is the case this serves. No counterpart in the reference. Layers loaded by
 * fl_gguf_load_moe_layer with FL_LAYOUT_TILED are declared by it and forgotten by fl_gguf_free_layer. */
int fl_register_tiled(FLCtx *, const void * base, size_t bytes);
/* forgets every declared range inside [base, base + bytes): call it before the memory is freed or holds ggml bytes */
int fl_unregister_tiled(FLCtx *, const void * base, size_t bytes);
/* RMSNorm (ggml semantics, eps) of n rows of D floats (D = 1024, 2048, 4096 or 7168), w may be NULL (ones) */
int fl_rmsnorm_dev(FLCtx *, const float * x, const float * w, float * y, int n, int D, float eps);
/* synthetic data on the device: IQ2_XXS matrices (qs uniform bytes, d = fp16(|N(0, sigma^2)|)) and normal floats */
int fl_synth_iq2xxs(FLCtx *, void * dst, size_t dst_stride, int R, int K, int nmat, int layout, uint64_t seed, uint64_t mat0, float sigma);
int fl_synth_normal(FLCtx *, float * dst, int64_t count, uint64_t seed, uint64_t stream, float mean, float sigma);
/* which = 0: exp, 1: sigmoid, 2: silu under the library's exp contract (device arrays) */
int fl_probe_exp(FLCtx *, const float * x, float * y, int64_t n, int which);

/* ---------------------------------------------------------------- additive: the model's GGUF shards
 * A tensor index over one or more GGUF files (ggml's container, versions 2 and 3): name -> file, absolute offset, ggml
 * type, dims; a later file's tensor of the same name replaces an earlier one. It replaces the reference's index built
 * with ggml's gguf API (src/server_core_fused.cpp:97-110); expert e of an expert tensor starts at offset + e *
 * expert_stride, expert_stride = ggml_row_size(type, ne[0]) * ne[1] (eng:305). Host only: no GPU needed. */
typedef struct FLGguf FLGguf;
typedef struct FLGgufTensor {
    int file;             /* index into the paths given to fl_gguf_open */
    int type;             /* ggml type code (F32 0, F16 1, Q2_K 10, Q3_K 11, Q5_K 13, Q6_K 14, IQ2_XXS 16, ...) */
    int fl_format;        /* the FL_* code of the type, -1 if this library has no kernel for it */
    int n_dims;
    int64_t ne[4];        /* ggml order: ne[0] = columns, ne[1] = rows, ne[2] = experts */
    uint64_t offset;      /* absolute byte offset in its file */
    uint64_t nbytes;      /* 0 for ggml types this index does not size */
    uint64_t row_bytes;   /* ggml_row_size(type, ne[0]) */
} FLGgufTensor;
/* NULL on failure, with the reason in err (errlen bytes, may be NULL) */
FLGguf * fl_gguf_open(const char * const * paths, int npaths, char * err, size_t errlen);
void fl_gguf_close(FLGguf *);
int fl_gguf_n_tensors(const FLGguf *);
const char * fl_gguf_tensor_name(const FLGguf *, int i);
/* FL_OK, FL_ERANGE when absent */
int fl_gguf_tensor(const FLGguf *, const char * name, FLGgufTensor * out);
int fl_gguf_tensor_at(const FLGguf *, int i, FLGgufTensor * out);
/* metadata: integer (u8..i64, bool), float (f32, f64), string; FL_ERANGE when absent, FL_EINVAL on a type mismatch */
int fl_gguf_get_int(const FLGguf *, const char * key, int64_t * out);
int fl_gguf_get_float(const FLGguf *, const char * key, double * out);
const char * fl_gguf_get_str(const FLGguf *, const char * key);
/* bytes [off, off + bytes) of a tensor's data into host memory */
int fl_gguf_read(const FLGguf *, const FLGgufTensor *, uint64_t off, uint64_t bytes, void * dst);

/* One MoE layer of the index (blk.<layer>.ffn_gate_inp / exp_probs_b / ffn_norm / ffn_{gate,up,down}_exps /
 * ffn_{gate,up,down}_shexp) made resident in HBM in one allocation. The router arrives F32 (ffn_gate_inp.weight, or
 * ffn_gate_inp_f16.weight widened exactly). layout FL_LAYOUT_TILED packs the IQ2_XXS matrices for fl_moe_layer /
 * fl_moe_layer_normed (K-quant ones stay as stored: call fl_set_layer_formats with fmt_down / fmt_sh_*);
 * FL_LAYOUT_GGML keeps every matrix as stored, for fl_moe / fl_wide_moe (the layer as the arena, ids = expert ids,
 * down_fmt = fmt_down) and fl_ffn_begin (FLW from L, fl_set_shared_formats with fmt_sh_*). Routed gate/up must be
 * IQ2_XXS, down IQ2_XXS, Q2_K or Q3_K, the shared expert IQ2_XXS or K-quants (FL_ESCOPE otherwise). */
typedef struct FLGgufLayer {
    FLMoeLayer L;
    const float * ffn_norm;                 /* [E] F32, device; NULL when the layer has no ffn_norm */
    int fmt_down, fmt_sh_gate, fmt_sh_up, fmt_sh_down;   /* FL_* codes of the files' types */
    uint64_t expert_stride[3];              /* gate, up, down bytes per expert */
    void * mem; size_t bytes;               /* the allocation (fl_gguf_free_layer) */
} FLGgufLayer;
int fl_gguf_load_moe_layer(FLCtx *, const FLGguf *, int layer, int layout, FLGgufLayer * out);
void fl_gguf_free_layer(FLGgufLayer *);

/* internal buffers of the last fl_moe_layer (device pointers, valid until the next call that resizes them) */
typedef struct FLDebug {
    const int8_t * xq; const float * xd;             /* Q8_K of x */
    const float * logits, * probs; const int * sel; const float * wts;
    const int * counts, * offsets, * perm, * inv, * act, * nact;
    const float * h; const int8_t * hq; const float * hd; /* [P+n][H]: per slot, shared rows at P.. (per-pass path) */
    const float * o;                                   /* [P+n][E] (per-pass path) */
    const float * g, * u;                              /* gate / up outputs when debug capture is on (per-pass path) */
    int n, P, topk;                                    /* topk: slots per row of the last call (the kept count) */
    int fused;                                         /* 1: the last call ran as the single-launch decode block, which
                                                        * keeps h and o internal (h .. u are NULL then) */
    int kernel;                                        /* the last call's decode launch: 0 none (per-pass or wide path),
                                                        * 1 the general block, 2 the one-token block organised by XCD,
                                                        * 3 that block launched by fl_ffn_begin on its own picks (fl_moe) */
} FLDebug;
int fl_debug(FLCtx *, FLDebug * out);
/* flags: bit 0 = capture the per-pass gate / up outputs (fl_debug's g, u); bit 1 = cap the y extent of the row-looping
 * combine / scatter grids at 7 (for every context of the process: tests of their row loops at small sizes); bit 2 = run
 * the per-pass decode's K-quant shared expert on the context's stream, not on its second stream beside the routed
 * launches (same results: tests compare the two) */
int fl_set_debug(FLCtx *, int flags);
/* decode batches (n <= 8, E 7168, H 2048) of fl_moe_layer: 2 (default) = the whole block as one regular launch of one
 * workgroup per CU (assumes nothing else occupies the CUs, as in a single-stream engine); 1 = the same kernel as a
 * cooperative launch (residency guaranteed by the runtime, ~18 us more per call at batch 1); 0 = one launch per pass.
 * Every device-wide wait of the single launch is bounded: if workgroups are not co-resident (another stream or process
 * holds CUs) a wait times out, the launch's outputs are invalid, and the code is reported twice -- by fl_sync, which
 * the caller must check before trusting any output of a mode-2 decode, and, without waiting, by the next
 * fl_moe_layer / fl_moe_layer_normed call on the context, which returns FL_EHIP until fl_sync has reported it. */
int fl_set_fused(FLCtx *, int mode);
/* single-token decode with all 8 picks kept, on a 256-CU device: 1 (default) = the single launch organised by XCD
 * (pick k's expert runs on the 32 CUs of XCD k, its down split by K-block among the four workgroups that produce each
 * h block), 0 = the general single-launch decode block. Both give bit-identical outputs. */
int fl_set_decode1(FLCtx *, int on);
/* batches above the decode sizes (n > 8, E 7168, H 2048): 1 (default) = the expert products as grouped GEMMs on the
 * matrix cores (no counterpart in the reference, whose wide path is tc_matvec per arena batch, src/fused_layer.cu:540-561);
 * 0 = the per-pass mat-vec kernels. Both give bit-identical outputs. */
int fl_set_prefill_mfma(FLCtx *, int on);

/* stage timing with HIP events on the context's stream: stages 0..5 = quant_x, router_logits, router_select, dispatch,
 * gate_up (with SwiGLU and Q8_K(h)), down (with the combine). fl_stage_ms waits for the profiled calls and returns their count (summed ms in ms[]). */
int fl_set_profile(FLCtx *, int on);
int fl_stage_ms(FLCtx *, double * ms, int nstage, int reset);

hipStream_t fl_stream(FLCtx *);
/* run on the caller's stream from now on (NULL = HIP's default stream); work queued on the previous stream finishes first */
int fl_set_stream(FLCtx *, hipStream_t s);
/* device -> host copy on the context's stream, waited (tests read internal buffers with it) */
int fl_d2h(FLCtx *, void * host, const void * dev, size_t bytes);
/* waits for the context's stream; FL_EHIP (with the code in fl_last_error) if a kernel reported a device-side failure
 * since the last fl_sync (decode block: a bounded wait timed out; MFMA prefill: a misaligned LDS base), then clears it */
int fl_sync(FLCtx *);
const char * fl_last_error(FLCtx *);
void fl_free(FLCtx *);

#ifdef __cplusplus
}
#endif
