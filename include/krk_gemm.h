/*
 * krk_gemm.h — C ABI of the MI355X (gfx950) skinny decode GEMM.
 *
 *   y[M, Nout] = epilogue( x[M, K] · W[N, K]ᵀ )      bf16 in, fp32 accumulate, bf16 out
 *
 * All operands are row-major bf16 (raw 16-bit bit patterns) in device memory.
 * Leading dimensions are in elements.  Nothing in this interface allocates,
 * synchronises or reads device memory on the host: every call enqueues its
 * kernels on `stream` and returns, so it may be recorded into a HIP graph.
 *
 * Reference interface replaced (willzeng274/kernel-rush-kawk, Python/Triton):
 *   engine/kernels/gemm.py:332-361  SkinnyMatmul.__init__/__call__  (C = A·Wᵀ)
 *   engine/kernels/gemm.py:298-329  SkinnyGateUp.__init__/__call__  (swiglu(A·Wgᵀ, A·Wuᵀ))
 *   engine/kernels/gemm.py:248-281  Gemv.__call__                   (M = 1 row dot products)
 *   engine/kernels/gemm.py:96-104, 160-170  _sum_kernel / _sum_gateup_kernel (split-K reduce)
 *   engine/kernels/gateup64.py:59-81        launch_gateup64 (caller-owned output, M = 64)
 * The reference exposes these as Python callables f(a, w) -> Tensor; the
 * Python mirror in kernel-rush-kawk_amd/kernels/gemm.py keeps that surface on
 * top of this ABI.
 */
#ifndef KRK_GEMM_H
#define KRK_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Epilogues applied to the fp32 accumulators before the bf16 store. */
enum {
    /* y = bf16(x·Wᵀ).  Nout = N. */
    KRK_EPILOGUE_NONE = 0,
    /* Fused gate/up + SwiGLU.  W rows [0, N/2) are the gate projection and rows
     * [N/2, N) the up projection (concatenation order of engine/model.py:116);
     * y[M, N/2] = bf16(bf16(silu_f32(bf16(g))) · bf16(u)), the three roundings
     * of engine/kernels/gemm.py:107-113 and engine/kernels/swiglu.py:14-24.
     * N must be even. */
    KRK_EPILOGUE_SILU_MUL = 1
};

/* Return codes (0 = success, negative = error; krk_last_error() explains). */
enum {
    KRK_OK = 0,
    KRK_ERR_INVALID = -1,     /* bad shape, stride, epilogue or null pointer */
    KRK_ERR_ALIGN = -2,       /* base pointer or leading dimension not 16-byte aligned */
    KRK_ERR_ALIAS = -3,       /* y overlaps x, W or the workspace */
    KRK_ERR_WORKSPACE = -4,   /* workspace missing or smaller than krk_gemm_workspace_bytes() */
    KRK_ERR_HIP = -5,         /* the HIP runtime rejected a launch */
    KRK_ERR_UNSUPPORTED = -6  /* a forced configuration this build does not provide */
};

/*
 * krk_gemm_bf16 — one projection call.
 *
 * Replaces SkinnyMatmul.__call__ (engine/kernels/gemm.py:346-361) and
 * SkinnyGateUp.__call__ (engine/kernels/gemm.py:314-329): the reference
 * allocates `c` and launches _skinny_kernel / _gateup_kernel plus the split-K
 * sum; here the caller owns y and the split-K workspace.
 *
 *   x          [M, K] bf16, row stride ldx >= K, ldx % 8 == 0, 16-byte aligned
 *   w          [N, K] bf16, row stride ldw >= K, ldw % 8 == 0, 16-byte aligned
 *   y          [M, Nout] bf16, row stride ldy >= Nout; must not overlap x, w or workspace
 *   M >= 1 (rows beyond 64 are processed in chunks of 64), N >= 1, K >= 8, K % 8 == 0
 *   epilogue   KRK_EPILOGUE_NONE or KRK_EPILOGUE_SILU_MUL
 *   workspace  device memory of at least krk_gemm_workspace_bytes(M, N, K, epilogue)
 *              bytes (may be NULL when that is 0).  It must be zero-filled once
 *              before its first use; every call leaves it zero-filled again.
 *              Calls that share one workspace must be ordered on one stream.
 *   stream     hipStream_t (NULL = the default stream)
 *
 * Results are deterministic: the same inputs and shape give bit-identical y.
 */
int krk_gemm_bf16(const void* x, int64_t ldx,
                  const void* w, int64_t ldw,
                  void* y, int64_t ldy,
                  int M, int N, int K, int epilogue,
                  void* workspace, size_t workspace_bytes,
                  void* stream);

/*
 * krk_gemm_workspace_bytes — split-K scratch needed by krk_gemm_bf16 for this
 * shape (0 when the chosen plan does not split K).  Replaces the per-object
 * partial-sum allocation of SkinnyMatmul.__init__ (engine/kernels/gemm.py:341)
 * and SkinnyGateUp.__init__ (engine/kernels/gemm.py:309).  Returns 0 for an
 * invalid shape as well; krk_gemm_bf16 then reports the shape error.
 */
size_t krk_gemm_workspace_bytes(int M, int N, int K, int epilogue);

/*
 * Kernel configuration.  Mirrors the per-candidate config dicts of the
 * reference (engine/kernels/gemm.py:284-288 GEMV_CONFIGS, :364-375 CONFIGS)
 * that SkinnyMatmul/Gemv are constructed from (gemm.py:251, 301, 333).
 * A field left at 0 takes the dispatcher's choice for this shape.
 */
enum {
    KRK_KERNEL_AUTO = 0,
    KRK_KERNEL_MFMA = 1,   /* bf16 MFMA 16x16x32 tiles, W fragments straight from HBM */
    KRK_KERNEL_VALU = 2,   /* dot2 row streaming in 512-k blocks (M <= 8); x in registers
                              (M <= 2) or staged once in LDS (M > 2) */
    KRK_KERNEL_MFMA_LDS = 3, /* bf16 MFMA 16x16x32, W and x rows streamed row-contiguously through LDS */
    KRK_KERNEL_STREAM = 5,  /* persistent bf16 MFMA: W through an LDS DMA ring, x held in registers */
    KRK_KERNEL_SLICE = 6    /* bf16 MFMA, every wave DMAs its own K chunks of W and x into a private
                               LDS ring (no barrier in the loop); plain epilogue, M <= 32 */
};

typedef struct krk_gemm_config {
    int kernel;   /* KRK_KERNEL_* */
    int m_tiles;  /* MFMA kernels: 16-row x tiles covering M (1..4); VALU: set from M
                     (x rows held: 1, 2, 4, 8), a caller's value is ignored */
    int n_tiles;  /* MFMA kernels: 16-row W tiles per workgroup (1, 2, 4; even with
                     SILU_MUL); VALU: W rows per wave (1, 2, 4; even with SILU_MUL) */
    int unroll;   /* MFMA: k-steps loaded per pipeline stage (2, 4, 8); VALU: 512-k
                     blocks in flight per row (2, 3, 4, 5, 7, 8, 10, 19, at most 48
                     loads in flight per lane); MFMA_LDS: stages in flight (2, or 3
                     when m_tiles + n_tiles <= 6); STREAM: ring depth in 512-k
                     stages (2..8, less at large M); SLICE: K chunks in flight per
                     wave (2 or 3) */
    int waves;    /* waves per workgroup (MFMA: 1, 2, 4; VALU: 1 to 8; MFMA_LDS and STREAM: 8) */
    int splits;   /* K partitions across workgroups, reduced in fixed order (1..32) */
    int k_chunk;  /* MFMA_LDS: k per pipeline stage, 256 or 512 (512 needs
                     m_tiles + n_tiles <= 4); SLICE: k per wave chunk, 64 or 128
                     (128 for up to 16 channels and M <= 16, 2 chunks in
                     flight); other kernels: ignored */
    int prologue; /* normed calls (krk_gemm_bf16_normed_config): 0 = fused into
                     the projection kernel where the configuration allows it
                     (krk_gemm_normed_fused), else a separate prologue kernel;
                     1 = always the separate prologue kernel.  Ignored by
                     plain calls. */
    int channels; /* MFMA_LDS: output channels per workgroup, a multiple of 8 up
                     to 16·n_tiles (8·n_tiles with SILU_MUL); 0 = the
                     dispatcher's choice (the plan's when the plan uses this
                     kernel and tile width, else all of them).
                     Fewer channels than the tiles hold leave the rest of the
                     last tile as padding (not loaded), so a shape can be cut
                     into exactly as many blocks as there are CUs.  SLICE:
                     output channels per workgroup, 1..32 (n_tiles and m_tiles
                     follow from channels and M); 0 = the plan's, else
                     N / 256 rounded up.  Other kernels: ignored. */
    int x_preload; /* MFMA_LDS: 1 = x rows loaded with every stage's weight
                     rows; 2 = x rows of the whole K loaded into registers
                     once, before the first stage, so the stage loop loads
                     weights only (k_chunk 512, K unsplit, K <= 4096 and
                     m_tiles <= 2, or K <= 9728 with m_tiles and n_tiles 1;
                     no token selection); 0 = the dispatcher's
                     choice (the plan's when the plan uses this kernel, else
                     1).  Other kernels: ignored. */
} krk_gemm_config;

/*
 * krk_gemm_plan — the configuration krk_gemm_bf16 uses for this shape (the
 * static shape -> kernel table that stands in for the reference's warm-up
 * pickers, engine/kernels/gemm.py:417-458, 461-498).  Returns KRK_OK or a
 * negative error for an invalid shape.
 */
int krk_gemm_plan(int M, int N, int K, int epilogue, krk_gemm_config* out);

/*
 * krk_gemm_candidates — the search space of a warm-up tuner for this shape:
 * every distinct configuration the library accepts from a fixed grid (VALU
 * rows per wave x waves x splits x blocks in flight for M <= 8, LDS-staged
 * MFMA tiles x stages
 * in flight x k per stage x splits, stream kernel depth x splits, register
 * MFMA tiles x splits), resolved as krk_gemm_bf16_config would resolve it,
 * krk_gemm_plan's configuration first.  Writes the first cap of them to out
 * and returns how many there are (negative on an invalid shape).  Stands in
 * for the GEMV_CONFIGS / CONFIGS lists the reference's pickers try
 * (engine/kernels/gemm.py:284, 364-375, used at 417-458).
 */
int krk_gemm_candidates(int M, int N, int K, int epilogue, krk_gemm_config* out, int cap);

/*
 * krk_gemm_config_workspace_bytes — as krk_gemm_workspace_bytes, for an
 * explicit configuration (0 fields filled from krk_gemm_plan).
 */
size_t krk_gemm_config_workspace_bytes(int M, int N, int K, int epilogue,
                                       const krk_gemm_config* cfg);

/*
 * krk_gemm_resolve — the configuration krk_gemm_bf16_config runs for `cfg`
 * (0 fields filled from krk_gemm_plan; NULL = the plan itself), or
 * KRK_ERR_UNSUPPORTED / KRK_ERR_INVALID with krk_last_error() explaining why
 * this build cannot run it.  The check the reference's constructors make
 * before a launch (SkinnyMatmul / SkinnyGateUp / Gemv.__init__,
 * engine/kernels/gemm.py:251-254, 301-311, 333-344), without launching.
 */
int krk_gemm_resolve(int M, int N, int K, int epilogue, const krk_gemm_config* cfg, krk_gemm_config* out);

/*
 * krk_gemm_bf16_config — krk_gemm_bf16 with an explicit configuration, the
 * counterpart of calling one candidate SkinnyMatmul(M, N, K, device, **cfg)
 * (engine/kernels/gemm.py:427-448).  Every configuration computes the same
 * function; they differ only in fp32 summation order.  Returns
 * KRK_ERR_UNSUPPORTED for a combination this build does not instantiate.
 */
int krk_gemm_bf16_config(const void* x, int64_t ldx,
                         const void* w, int64_t ldw,
                         void* y, int64_t ldy,
                         int M, int N, int K, int epilogue,
                         const krk_gemm_config* cfg,
                         void* workspace, size_t workspace_bytes,
                         void* stream);

/*
 * krk_gemm_bf16_normed — a projection with the residual-add + RMSNorm
 * prologue fused in front:
 *
 *   xout = bf16(x + d)
 *   n    = bf16(bf16(xout · rsqrt(mean(xout²) + eps)) · w_norm)   (mean in fp32)
 *   y    = epilogue(n · Wᵀ)
 *
 * Replaces the reference's normed call f(x, y, w_norm, xout, w) that
 * pick_normed returns (engine/kernels/gemm.py:501-560), i.e.
 * SkinnyMatmul.__call__(a, w, norm=(y, w_norm, xout, eps)) (gemm.py:346-361)
 * and SkinnyGateUp.__call__(a, wg, wu, norm=...) (gemm.py:314-329); the
 * rounding points are those of gemm.py:21-51 and add_rmsnorm.py:15-29.  `d`
 * is the reference's `y` (the branch output added to the residual x).
 *
 *   x, d       [M, K] bf16, strides ldx, ldd (multiples of 8, 16-byte aligned)
 *   w_norm     [K] bf16 RMSNorm gain; eps >= 0
 *   xout       [M, K] bf16 output, stride ldxo; may not overlap x, d, w_norm, W, y
 *   w, y, M, N, K, epilogue, stream   as krk_gemm_bf16 (K <= 16384)
 *   workspace  krk_gemm_normed_workspace_bytes(M, N, K, epilogue, NULL) bytes;
 *              its split-K counters must be zero before first use (every call
 *              leaves them zero); the rest is scratch.
 *
 * Fused (one launch; krk_gemm_normed_fused tells when), K unsplit: a VALU
 * configuration at the depth that covers K = 2560 in one pass, with a wave
 * per 512-k block (K <= 512·waves); or an MFMA_LDS configuration with
 * k_chunk 512, K <= 2560, m_tiles <= 2 (M <= 32) and n_tiles <= 2 (unroll 2
 * when both are 2).  Every
 * workgroup then normalises the rows of x itself while its first weight
 * loads are in flight (no workgroup waits for another; workgroup 0 writes
 * xout).
 * Otherwise (and with prologue = 1) a one-workgroup-per-row prologue kernel
 * writes xout and the normalised rows into the workspace, then the
 * projection runs; in front of a STREAM projection of at most 64 rows the
 * rows go in that kernel's MFMA fragment order (padded to 16-row tiles and
 * whole 512-k stages), so that it loads them as whole 1 KB runs and skips
 * their trip through LDS.  Both use the rounding points above.  With
 * cfg == NULL the call uses krk_gemm_normed_plan.
 */
int krk_gemm_bf16_normed(const void* x, int64_t ldx, const void* d, int64_t ldd,
                         const void* w_norm, float eps, void* xout, int64_t ldxo,
                         const void* w, int64_t ldw, void* y, int64_t ldy,
                         int M, int N, int K, int epilogue,
                         void* workspace, size_t workspace_bytes, void* stream);

/* krk_gemm_bf16_normed with an explicit configuration (as krk_gemm_bf16_config). */
int krk_gemm_bf16_normed_config(const void* x, int64_t ldx, const void* d, int64_t ldd,
                                const void* w_norm, float eps, void* xout, int64_t ldxo,
                                const void* w, int64_t ldw, void* y, int64_t ldy,
                                int M, int N, int K, int epilogue, const krk_gemm_config* cfg,
                                void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of krk_gemm_bf16_normed(_config); cfg may be NULL (the
 * plan).  0 for an invalid shape or configuration. */
size_t krk_gemm_normed_workspace_bytes(int M, int N, int K, int epilogue, const krk_gemm_config* cfg);

/* 1 when the normed call for this shape and configuration (NULL = the
 * normed plan) runs the prologue inside the projection kernel, 0 when it
 * launches the separate prologue kernel first, negative on an invalid
 * shape/config. */
int krk_gemm_normed_fused(int M, int N, int K, int epilogue, const krk_gemm_config* cfg);

/* The configuration krk_gemm_bf16_normed uses (the normed plan): fused where
 * that measured fastest (qkv at M <= 4, gate_up and lm_head at M <= 2 of
 * Qwen3-4B, all on the VALU kernel), else the plain plan with
 * prologue = 1.  Like krk_gemm_plan it
 * replaces the configuration pick_normed settles on
 * (engine/kernels/gemm.py:501-560).  KRK_OK or a negative code. */
int krk_gemm_normed_plan(int M, int N, int K, int epilogue, krk_gemm_config* out);

/*
 * krk_add_rms_norm_bf16 — the stand-alone prologue: xout = bf16(x + d) and
 * out = bf16(bf16(xout · rstd) · w_norm) per row, one workgroup per row.
 * Replaces add_rms_norm (engine/kernels/add_rmsnorm.py:32-43), which the
 * reference's unfused path launches in front of a plain projection
 * (engine/model.py:161-171).  K <= 16384; xout may be x itself (same pointer
 * and stride: in place, as the reference allows); otherwise xout and out may
 * not overlap each other or the inputs.
 */
int krk_add_rms_norm_bf16(const void* x, int64_t ldx, const void* d, int64_t ldd,
                          const void* w_norm, float eps, void* xout, int64_t ldxo,
                          void* out, int64_t ldo, int M, int K, void* stream);

/*
 * krk_gemm_bf16_select — the lm_head projection followed by token selection:
 * idx[m][0..k) = indices of the k largest bf16 logits bf16(x[m]·W[n]ᵀ) of
 * row m, largest first, equal values at the lower index first (NaN above
 * +inf, -0 equal to +0).  For k = 1 behind a VALU, LDS-staged MFMA or
 * stream projection, and for k > 1 behind a stream projection of up to 16
 * rows (krk_gemm_select_fused), the projection's epilogue reduces its
 * outputs to one key per row and workgroup and the logits are not written
 * unless y is given; otherwise the plain projection writes the logits (to y,
 * or to the workspace) and a selection kernel reads them back.  Either way
 * the call is two kernels on one stream.
 *
 * Replaces `logits.argmax(dim=-1)` (k = 1; engine/engine.py:196,
 * engine/model.py:365; lowest index on ties, OPTIMIZATION_GUIDE.md:213) and
 * `torch.topk(logits, k).indices` (engine/recycle.py:170, k = 8) after the
 * lm_head call of engine/model.py:209.
 *
 *   x, w, M, N, K   as krk_gemm_bf16 (plain epilogue)
 *   y               [M, N] bf16 logits, stride ldy >= N, or NULL to skip them
 *   k               1..8 (<= N)
 *   idx             [M, k] int64 output, 8-byte aligned
 *   vals            [M, k] bf16 values of the selected logits (a NaN as the
 *                   canonical quiet NaN 0x7fc0), or NULL
 *   workspace       krk_gemm_select_workspace_bytes(M, N, K, k, NULL) bytes,
 *                   256-byte aligned, zero-filled before first use; every call
 *                   leaves its counters zero
 */
int krk_gemm_bf16_select(const void* x, int64_t ldx, const void* w, int64_t ldw,
                         void* y, int64_t ldy, int M, int N, int K, int k,
                         int64_t* idx, void* vals,
                         void* workspace, size_t workspace_bytes, void* stream);

/* krk_gemm_bf16_select with an explicit projection configuration (any
 * configuration krk_gemm_bf16_config accepts for the plain epilogue). */
int krk_gemm_bf16_select_config(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                void* y, int64_t ldy, int M, int N, int K, int k,
                                int64_t* idx, void* vals, const krk_gemm_config* cfg,
                                void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of a selecting call (cfg may be NULL: the plan); 0 for an
 * invalid shape, k or configuration. */
size_t krk_gemm_select_workspace_bytes(int M, int N, int K, int k, const krk_gemm_config* cfg);

/* The projection configuration krk_gemm_bf16_select uses for this shape and k. */
int krk_gemm_select_plan(int M, int N, int K, int k, krk_gemm_config* out);

/* 1 if the selection is fused into the projection's epilogue (the logits are
 * then written only when y is given), 0 if the projection writes the logits
 * and a selection kernel reads them, negative on an invalid shape, k or
 * configuration (cfg may be NULL: the plan). */
int krk_gemm_select_fused(int M, int N, int K, int k, const krk_gemm_config* cfg);

/*
 * krk_gemm_bf16_noalloc — krk_gemm_bf16 without a workspace argument, for
 * callers that cannot allocate device memory (code under HIP graph capture
 * that may not call hipMalloc, tight serving loops, harnesses that forbid
 * allocation).  This entry point has no counterpart in the reference; it
 * exists for those callers, which cannot allocate.
 *
 * The split-K counters and partials live in a static device array of
 * KRK_NOALLOC_SCRATCH_BYTES that the library holds on every GPU it runs on
 * until the process ends (counters in its first KRK_NOALLOC_COUNTER_BYTES).
 * A plan whose partials or counters do not fit returns KRK_ERR_WORKSPACE
 * (every Qwen3-4B projection plan at M <= 64 fits: at most 1.97 MB).  The
 * call allocates nothing and never synchronises.  All calls on one GPU share
 * that GPU's array: calls that may overlap in time on one GPU (different
 * streams, or several host threads) race and must not be issued; calls
 * ordered on one stream are fine.
 */
#define KRK_NOALLOC_SCRATCH_BYTES (4u << 20)
#define KRK_NOALLOC_COUNTER_BYTES (64u << 10)
int krk_gemm_bf16_noalloc(const void* x, int64_t ldx,
                          const void* w, int64_t ldw,
                          void* y, int64_t ldy,
                          int M, int N, int K, int epilogue,
                          void* stream);

/*
 * ABI identification, for bindings that lay out krk_gemm_config themselves
 * (a ctypes / cgo / JNI stub).  No counterpart in the reference: its kernels
 * are Python objects with no binary interface.
 *
 * krk_abi_version — KRK_ABI_VERSION of the built library.  The version moves
 *   whenever a declaration or the krk_gemm_config layout changes (version 3:
 *   the ten-int krk_gemm_config above, prologue/channels/x_preload added to
 *   version 1's seven ints; version 4: kernel KRK_KERNEL_SLICE, which a
 *   plan or a candidate list may now name).
 * krk_gemm_config_size — sizeof(krk_gemm_config) in the built library.  A
 *   binding must check both at load time and refuse a mismatch: a config
 *   array of another layout would be over- or under-read.
 */
#define KRK_ABI_VERSION 4
int krk_abi_version(void);
size_t krk_gemm_config_size(void);

/*
 * krk_last_error — text of the last error raised on the calling thread by
 * any krk_* function ("" if none).  Stands in for the ValueError messages of
 * engine/kernels/gateup64.py:63-74 and engine/kernels/gemm.py:253-254.
 */
const char* krk_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* KRK_GEMM_H */
