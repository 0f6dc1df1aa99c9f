/*
 * trellis_amd.h — C ABI of the MI355X (gfx950) trellis packed-linear library.
 *
 * Plain C: device pointers, sizes and an opaque stream handle (a hipStream_t passed
 * as void*; NULL is the default stream). No torch or HIP types appear here.
 *
 * Semantics follow the reference's packed linear: y = restore(decode(bits)) @ x, with
 * the incoherence-processing transforms folded onto the activations
 * (web/packed.js:163-182):
 *     xf = Hb_k(isc_scaled * su * x);  t = Zq @ xf;  y = sv * osc * Hb_n(t)
 * where Zq is decoded from the packed K-bit trellis stream (src/trellis/qtip.py:82-110,
 * web/kernels.js:115-122), Hb_d is the normalized block-diagonal Sylvester Hadamard
 * with block fit(d,128) (qtip.py:200-223) and isc_scaled = f32(isc) * scale, folded at
 * load as web/packed.js:51-52 does.
 *
 * Conventions
 *  - The caller owns every buffer. No call allocates device memory.
 *  - Calls are ordered on `stream` and never synchronize the host.
 *  - Calls that share one workspace must not overlap (use one workspace per stream).
 *  - Errors are returned as trellis_status codes; trellis_strerror() names them.
 */
#ifndef TRELLIS_AMD_H
#define TRELLIS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Codebook ids (qtip.py:32-56). The reference manifest has no codebook field and
 * hard-codes MCG (export_packed.py:42); absent means TRELLIS_CB_MCG. */
enum trellis_codebook {
  TRELLIS_CB_MCG = 0,   /* x*0xCBAC1FED, lop3, fp16 halves summed in fp32 (qtip.py:48-53) */
  TRELLIS_CB_3INST = 1, /* x*89226354+64248484, lop3, fp16 halves (qtip.py:40-45) */
  TRELLIS_CB_1MAD = 2   /* x*34038481+76625530, byte sum, (y-510)/147.800537109375 (qtip.py:32-37) */
};

enum trellis_dtype { TRELLIS_F32 = 0, TRELLIS_F16 = 1 };

typedef enum trellis_status {
  TRELLIS_OK = 0,
  TRELLIS_ERR_NULL = 1,        /* a required pointer is NULL */
  TRELLIS_ERR_SHAPE = 2,       /* n or k not a positive multiple of 16 */
  TRELLIS_ERR_BLOCK = 3,       /* Hadamard block not a power of 2 in [16,128] dividing the dim */
  TRELLIS_ERR_K = 4,           /* bits/weight outside {2,3,4} */
  TRELLIS_ERR_V = 5,           /* weights per trellis step other than 1 or 2 */
  TRELLIS_ERR_CODEBOOK = 6,    /* unknown codebook id */
  TRELLIS_ERR_NWORDS = 7,      /* nwords != 256*K/32 */
  TRELLIS_ERR_ALIGN = 8,       /* bits not 16-byte aligned, or a stride too small */
  TRELLIS_ERR_DTYPE = 9,       /* unsupported x/y dtype */
  TRELLIS_ERR_WORKSPACE = 10,  /* workspace missing or smaller than trellis_workspace_bytes */
  TRELLIS_ERR_BATCH = 11,      /* batch < 1 */
  TRELLIS_ERR_RANGE = 12,      /* tile range outside the matrix */
  TRELLIS_ERR_LAUNCH = 13,     /* the HIP runtime rejected a launch */
  TRELLIS_ERR_GROUP = 14,      /* group of 0 or more than 8 linears, or mixed K / V / codebook */
  TRELLIS_ERR_FLAGS = 15,      /* unknown bits in the flags of an _ex call */
  TRELLIS_ERR_SCRATCH = 16,    /* a _noalloc call needs more than TRELLIS_NOALLOC_SCRATCH_BYTES */
  TRELLIS_ERR_CAPTURE = 17     /* the first _noalloc call on a device made under stream capture */
} trellis_status;

/* Flags of trellis_packed_linear_ex / trellis_packed_linear_group_ex. */
enum trellis_flags {
  /* The batched MFMA kernel only (calls that run the exact decode-GEMV, batch 1 to 4 and
   * narrow groups at 5 to 16, ignore it): round each decoded codebook value once to fp16
   * (hi + lo in one fp16 add, i.e. the reference's exact fp32 sum, qtip.py:28-29, rounded
   * to nearest) and multiply it by the fp16 activation once, instead of the exact (hi, lo)
   * pair against a duplicated activation: half the MFMAs and half the activation bytes of
   * the batched kernel. Max rel err against the exact path ~2-3e-4 (MCG, 3INST; 1MAD
   * values are exact fp16 integers either way). The reference's Triton codebook adds the
   * halves in fp16 the same way (src/trellis/viterbi_triton.py:29-31). */
  TRELLIS_MMA_F16 = 1
};

/* One packed trellis linear as the loader record holds it (web/packed.js:53-62,
 * 93-103): device pointers to the packed words and f32 metadata. */
typedef struct trellis_desc {
  const uint32_t *bits;      /* u32 [ntiles * nwords], tile = (row/16)*tiles_in + col/16 */
  const float *su;           /* [k_in]  input-dim signs */
  const float *sv;           /* [n_out] output-dim signs */
  const float *isc_scaled;   /* [k_in]  f32(isc) * scale */
  const float *osc;          /* [n_out] per-out-channel scale */
  int32_t n_out;             /* rows, multiple of 16 */
  int32_t k_in;              /* cols, multiple of 16 */
  int32_t K;                 /* bits per weight: 2, 3 or 4 */
  int32_t V;                 /* weights per trellis step: 1 (the reference), or 2: the tile's
                              * stream read as 128 steps of 2K bits, step u at stream bit
                              * (127-u)*2K; the step's state gives weight 2u from the
                              * codebook's first LCG iterate and weight 2u+1 from the second
                              * (no reference counterpart: qtip.py:4 has V=1 only) */
  int32_t codebook;          /* enum trellis_codebook */
  int32_t block_in;          /* fit(k_in, 128) */
  int32_t block_out;         /* fit(n_out, 128) (web/packed.js:173-176) */
  int32_t nwords;            /* 256*K/32 words per tile */
} trellis_desc;

/* Number of workspace bytes trellis_packed_linear needs for this layer and batch.
 * The workspace must be zero-filled once when allocated; every call leaves its
 * counters at zero again. It belongs to one layer (or one group): its counters sit in a
 * header laid out by the members' shapes alone, so calls at any batch size may share it
 * (sized for the largest), but another layer's calls may not. Replaces the per-call scratch f32buf allocations of
 * web/packed.js:165-180. */
int trellis_workspace_bytes(const trellis_desc *W, int batch, size_t *bytes);

/* y[b, :] = W_hat @ x[b, :] for b < batch. Replaces PackedOps.linear
 * (web/packed.js:163-182) and its Python mirror linear() (scripts/run_packed_headless.py:87-99).
 *   x: [batch, k_in] with row stride ldx elements, dtype x_dtype (f16 or f32)
 *   y: [batch, n_out] with row stride ldy elements, dtype y_dtype (f16 or f32)
 * Batch 1 to 4 runs one decode-GEMV launch (gemv_kernel, x fold fused; the batch rows
 * ride the MFMA's columns), and so does batch 5 to 16 when that launch's work items fit one
 * round on the CUs. Other calls run the x fold once (xfold_kernel), then the
 * decode-once batched kernel (bgemm_kernel: each weight tile decoded once per 16 to 128
 * batch columns, as the launch plan chooses, and fed to exact fp16 MFMAs), and, when the
 * launch plan splits k, the slice
 * reduction and output fold (bfold_kernel). */
int trellis_packed_linear(const trellis_desc *W, const void *x, int64_t ldx, int batch,
                          int x_dtype, void *y, int64_t ldy, int y_dtype, void *workspace,
                          size_t ws_bytes, void *stream);

/* trellis_packed_linear with flags (enum trellis_flags; 0 = trellis_packed_linear). No
 * reference counterpart: the precision choice of the batched MFMAs. The workspace size
 * from trellis_workspace_bytes covers every flag. */
int trellis_packed_linear_ex(const trellis_desc *W, const void *x, int64_t ldx, int batch,
                             int x_dtype, void *y, int64_t ldy, int y_dtype, void *workspace,
                             size_t ws_bytes, int flags, void *stream);

/* Several independent packed linears in ONE launch (no reference counterpart: the
 * reference dispatches every linear separately, web/model.js:80-100). Intended for the
 * linears of a decoder block that share an input (q/k/v, gate/up) or any set whose
 * inputs are ready together. Up to 8 linears, all with the same K and codebook; each
 * has its own x[i] (row stride ldx[i]) and y[i] (row stride ldy[i]). Same semantics per
 * linear as trellis_packed_linear. */
int trellis_workspace_bytes_group(const trellis_desc *const *W, int count, int batch,
                                  size_t *bytes);
int trellis_packed_linear_group(const trellis_desc *const *W, int count, const void *const *x,
                                const int64_t *ldx, int batch, int x_dtype, void *const *y,
                                const int64_t *ldy, int y_dtype, void *workspace,
                                size_t ws_bytes, void *stream);
/* trellis_packed_linear_group with flags (enum trellis_flags), as trellis_packed_linear_ex. */
int trellis_packed_linear_group_ex(const trellis_desc *const *W, int count,
                                   const void *const *x, const int64_t *ldx, int batch,
                                   int x_dtype, void *const *y, const int64_t *ldy, int y_dtype,
                                   void *workspace, size_t ws_bytes, int flags, void *stream);

/* No counterpart in the reference: for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * semantics, validation and kernels as trellis_packed_linear_group_ex, but no workspace
 * argument: the workspace is a static device array of TRELLIS_NOALLOC_SCRATCH_BYTES that
 * the library holds on every GPU it runs on until the process ends. The call allocates
 * nothing (no hipMalloc, no allocating library routine). A call whose plan needs more
 * workspace than that returns TRELLIS_ERR_SCRATCH (the Qwen3-8B block linears fit up to a
 * batch of 128 rows). Every call on a GPU shares that GPU's array: the split-K counters a
 * call needs are zeroed by a small kernel at its start, and calls that overlap on one GPU
 * (on different streams, or from several threads) race and must be serialized by the
 * caller. The first call on each device looks up that device's address of the array
 * (hipGetSymbolAddress); it must not be made under stream capture, and returns
 * TRELLIS_ERR_CAPTURE if it is. Later calls may be captured. */
#define TRELLIS_NOALLOC_SCRATCH_BYTES (32u << 20)
int trellis_packed_linear_group_noalloc(const trellis_desc *const *W, int count,
                                        const void *const *x, const int64_t *ldx, int batch,
                                        int x_dtype, void *const *y, const int64_t *ldy,
                                        int y_dtype, int flags, void *stream);

/* Decode z-space tiles [tile_begin, tile_begin+ntiles) to fp32, 256 values per tile in
 * tile order t = (row%16)*16 + col%16. The bit-exact probe of the decode: restates
 * decode_window over the packed stream (qtip.py:82-110, web/kernels.js:115-122) with the
 * codebooks of qtip.py:32-53, using the same window/codebook code as the matmul
 * kernels. */
int trellis_decode_tiles(const trellis_desc *W, uint32_t tile_begin, uint32_t ntiles,
                         float *out, void *stream);

/* Embedding rows with the full restore: out[t, :] = W_hat[tokens[t], :] for t < ntok.
 * Replaces PackedOps.embedRow / DECODE_EMBED (web/packed.js:137-146,
 * web/kernels.js:192-249), which decodes one token per dispatch; here ntok tokens per call.
 *   tokens: device int32 [ntok]; an id outside [0, n_out) yields a row of zeros
 *   out: [ntok, k_in] with row stride ldo elements, dtype out_dtype (f16 or f32)
 * Each token decodes the block_out x k_in weights of its row's Hadamard block once. */
int trellis_embed_rows(const trellis_desc *W, const int32_t *tokens, int ntok, void *out,
                       int64_t ldo, int out_dtype, void *stream);

/* Tail-biting trellis encode of z-space tiles (the encoder side of the format): the
 * counterpart of the reference's Triton encoder viterbi_tb_triton and of qtip.viterbi_tb
 * (src/trellis/viterbi_triton.py:34-129, src/trellis/qtip.py:124-196; L = 16, T = 256,
 * V = 1, QTIP's two-pass tail-biting). For each tile, the minimum squared-error path of
 * the K-bit bitshift trellis under `codebook`:
 *   w:    device f32 [ntiles][256] targets in tile order t = (row%16)*16 + col%16
 *   bits: device u32 [ntiles][8K] packed symbols in the reference's reversed stream
 *         layout (scripts/export_packed.py:27-35), ready for trellis_desc.bits
 *   dq:   device f32 [ntiles][256] codebook values of the chosen states, or NULL
 * The DP is exact (every state of every step; ties keep the smallest candidate and the
 * smallest final edge). The workspace (trellis_encode_workspace_bytes, 256-byte aligned)
 * holds the backpointers of the tiles in flight; it needs no initialisation. */
int trellis_encode_workspace_bytes(int K, uint32_t ntiles, size_t *bytes);
int trellis_encode_tiles(const float *w, uint32_t ntiles, int K, int codebook, uint32_t *bits,
                         float *dq, void *workspace, size_t ws_bytes, void *stream);

/* Human-readable name of a status code. */
const char *trellis_strerror(int status);

/* Library version string (no reference counterpart). */
const char *trellis_version(void);

#ifdef __cplusplus
}
#endif

#endif /* TRELLIS_AMD_H */
