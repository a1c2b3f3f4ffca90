/*
 * okf_quant.h -- C ABI of the MI355X (gfx950) quantized weight x activation
 * path: fused dequantize-and-dot for GGUF Q8_0, Q4_K, IQ2_XXS and the Bonsai
 * ternary Q2_0 blocks, plus Q4_0, IQ4_NL, Q5_K, Q6_K, IQ4_XS, IQ2_XS, IQ2_S,
 * IQ3_XXS, IQ3_S, IQ1_S, IQ1_M, Q2_K and Q3_K, and plain f32 / f16 / bf16
 * weights (whose kernels take K a multiple of 32).
 *
 * This ABI is the drop-in boundary for the reference's GPU dispatch surface
 * (LLM/Base/MetalEnc.swift) and the weight reference it takes
 * (LLM/Base/MetalContext.swift:4-11).  A Swift caller imports it through
 * include/module.modulemap.
 *
 * Conventions (same as the reference kernels, LLM/metal/Kernels.metal):
 *   - W has M rows of K weights; row m's blocks are contiguous at byte
 *     m * rowBytes(K), starting at base + off (GGUF dims = [K, M]).
 *   - x / X are fp32, row-major X[N][K]; outputs are fp32 Y[N][M]
 *     (out[n * M + m], Kernels.metal:112).
 *   - Every pointer passed to okf_gemv / okf_gemm / okf_dequant_row is device
 *     memory owned by the caller.  Calls are asynchronous on the context's
 *     stream (okf_sync waits); a context is used by one thread at a time.
 *   - Nothing aborts: each entry point returns an okf_status.
 */
#ifndef OKF_QUANT_H
#define OKF_QUANT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes.  The reference turns these conditions into fatalError /
 * precondition (MetalEnc.swift:109-113, :144-146, :268-269) or a GPUGate
 * verdict (LLM/Base/MetalGates.swift:130-142). */
typedef enum {
    OKF_OK = 0,
    OKF_E_TYPE = 1,     /* ggml type has no kernel here */
    OKF_E_SHAPE = 2,    /* K not a whole number of blocks, zero size, misalignment */
    OKF_E_HIP = 3,      /* a HIP runtime call failed (see okf_last_hip_error) */
    OKF_E_INJECTED = 4, /* fault injected by okf_set_fault_rate */
    OKF_E_ARG = 5,      /* null pointer or bad argument */
    OKF_E_NODEV = 6,    /* detached context (device -1): nothing can run */
    OKF_E_IO = 7,       /* a file could not be opened or mapped */
    OKF_E_FORMAT = 8,   /* a malformed GGUF file (GGUFErr.parse) */
    OKF_E_NOTFOUND = 9, /* no such tensor or key */
    OKF_E_TIMEOUT = 10  /* a one-launch FFN's grid barrier gave up (its outputs hold NaN);
                           reported by the next okf_sync or okf_ffn on the context */
} okf_status;

/* ggml type ids, LLM/Base/GGUF.swift:3-14 */
enum {
    OKF_TYPE_Q4_0 = 2,
    OKF_TYPE_Q8_0 = 8,
    OKF_TYPE_IQ4_NL = 20,
    OKF_TYPE_Q4_K = 12,
    OKF_TYPE_Q5_K = 13,
    OKF_TYPE_Q6_K = 14,
    OKF_TYPE_IQ4_XS = 23,
    OKF_TYPE_IQ2_XS = 17,
    OKF_TYPE_IQ3_XXS = 18,
    OKF_TYPE_IQ1_S = 19,
    OKF_TYPE_IQ3_S = 21,
    OKF_TYPE_IQ2_S = 22,
    OKF_TYPE_IQ1_M = 29,
    OKF_TYPE_Q2_K = 10,
    OKF_TYPE_Q3_K = 11,
    OKF_TYPE_F32 = 0,
    OKF_TYPE_F16 = 1,
    OKF_TYPE_BF16 = 30,
    OKF_TYPE_IQ2_XXS = 16,
    OKF_TYPE_Q2_0 = 42
};

typedef struct okf_ctx okf_ctx;

/* A quantized tensor in device memory.  Replaces GGUFTensor + WeightRef
 * {buf, local u64 off} (LLM/Base/GGUF.swift:49-57,
 * LLM/Base/MetalContext.swift:4-11): the 64-bit off lets one base address a
 * weight window larger than 4 GB (Kernels.metal:22-24). */
typedef struct {
    const void *base;
    uint64_t off;
    uint32_t K;        /* weights per row (dims[0]) */
    uint32_t M;        /* rows (dims[1]) */
    int32_t ggml_type;
} okf_weight;

/* Replaces MetalContext.init (MetalContext.swift:58-80): binds a device,
 * creates the stream and uploads the IQ2_XXS grid.  device = -1 makes a
 * detached context that validates arguments and injects faults but runs
 * nothing (OKF_E_NODEV), for host-only tests. */
int okf_ctx_create(int device, okf_ctx **out);
int okf_ctx_destroy(okf_ctx *ctx);

/* The hipStream_t the context launches on (for events / interop). */
int okf_ctx_stream(okf_ctx *ctx, void **stream);

/* Allocates the context's scratch up front, the counterpart of the
 * reference's engine-owned buffers (MetalContext.swift:216-236; MetalEnc
 * allocates nothing on the hot path): the fp16 activation copy of a Q4_K
 * tile GEMM with N * K <= gemm_nk, and the pairs and row counters of
 * okf_argmax_rows over up to argmax_rows rows of argmax_n values.  Afterwards
 * no call allocates or synchronises; one that needs more scratch than
 * reserved returns OKF_E_SHAPE.  Nor does any call allocate while the
 * context's stream is being captured into a graph.  (The tile GEMM of the other formats uses
 * the same scratch for its K-split partials and fp16 activations where it
 * fits, and otherwise runs without them: one K range, or the activations
 * rounded per tile; the K split changes only the order of the fp32 sums.)
 * Without it the scratch grows on demand (hipMalloc after draining the
 * stream). */
int okf_ctx_reserve(okf_ctx *ctx, uint64_t gemm_nk, uint32_t argmax_n, uint32_t argmax_rows);

/* GGUF.rowByteCount (LLM/Base/GGUF.swift:160-188) for the types above: n a
 * whole number of blocks, or any n for f32 / f16 / bf16. */
int okf_row_bytes(int32_t ggml_type, uint64_t n, uint64_t *out);

/* MetalEnc.gemv (MetalEnc.swift:84-93): y[M] = W x[K].
 * Q4_K needs base + off 16-byte aligned; x must be 16-byte aligned. */
int okf_gemv(okf_ctx *ctx, const okf_weight *w, const float *x, float *y);

/* MetalEnc.siluMul (MetalEnc.swift:921, kernel silu_mul,
 * LLM/metal/Kernels.metal:3280-3285) then MetalEnc.gemv on its output, the
 * FFN down projection (LLM/Qwen/QwenMetalEngine.swift:924-928), as one
 * launch: y[M] = W (silu(gate) * up), silu(x) = x / (1 + exp(-x)) in fp32.
 * Unlike the reference's in-place siluMul, gate is left unchanged. */
int okf_gemv_silu(okf_ctx *ctx, const okf_weight *w, const float *gate, const float *up, float *y);

/* The gate and up projections of the reference's FFN with its SiLU
 * (LLM/Qwen/QwenMetalEngine.swift:918-925: MetalEnc.parallel { gemv(gate);
 * gemv(up) } then the in-place siluMul(gate, up)): u = W_up x,
 * g = silu(W_gate x) * u.  One launch when gate and up share a format (each
 * workgroup computes the same rows of both); gate and up have the same K
 * and M; x, g, u 16-byte aligned. */
int okf_gemv_gate_up(okf_ctx *ctx, const okf_weight *gate, const okf_weight *up, const float *x, float *g,
                     float *u);

/* The FFN block of the reference's engines (LLM/Qwen/QwenMetalEngine.swift:
 * 918-929: MetalEnc.parallel { gemv(gate); gemv(up) }, siluMul, gemv(down)):
 * u = W_up x, g = silu(W_gate x) * u, y = W_down g.  As in the reference,
 * whose siluMul works in place on the gate buffer, g holds silu(gate) * up
 * after the call.  With Q2_0 gate, up and down (gate / up K <= 4096, M <=
 * 8192) one launch: gate and up, a grid-wide barrier, then down, every
 * weight requested at the start.  That launch needs one workgroup resident
 * on every CU at once: work that a caller keeps running on other streams of
 * the same GPU can delay it, and a barrier that waits past its bound
 * (about 0.3 s) leaves NaN in every y row of that launch rather than wait
 * forever; the next okf_sync then returns OKF_E_TIMEOUT once (or, with no
 * okf_sync between, the next okf_ffn returns it and launches nothing)
 * (OKF_FFN_FUSED=0 at okf_ctx_create selects the two launches).  At gate / up
 * 6144 x 2048 (the Bonsai FFN) two launches on the integer matrix cores are
 * faster and are the default (OKF_FFN_FUSED=2 keeps the one launch, which then
 * also computes on the matrix cores; OKF_FFN_MFMA=0 its VALU form; the same
 * outputs within 1e-5).  Otherwise two launches when gate and up
 * share a format: one grid whose workgroups each compute the same rows of
 * gate and up and form silu(g) * u there, then the down projection.
 * down->K must equal gate->M; x, g, u 16-byte aligned. */
int okf_ffn(okf_ctx *ctx, const okf_weight *gate, const okf_weight *up, const okf_weight *down, const float *x,
            float *g, float *u, float *y);

/* MetalEnc.siluMul (MetalEnc.swift:921): a[i] = silu(a[i]) * b[i], n values. */
int okf_silu_mul(okf_ctx *ctx, float *a, const float *b, uint32_t n);

/* MetalEnc.gemm (MetalEnc.swift:241-289): Y[N][M] = X[N][K] W^T.  Dispatch
 * policy as the reference: N == 1 -> gemv; 2 <= N <= 5 -> narrow (one weight
 * pass serving all N columns, gemmNarrow / gemmNarrowIQ :176-239);
 * N > 5 -> MFMA tile GEMM (gemmTiled / iqGemmTiled, :354-400; a grid of
 * fewer than two tiles a CU splits K over workgroups, partials added in K
 * order), except that a small N past 5 (up to a per-format bound, 5..16
 * columns, where measured faster than the tile) runs as consecutive narrow
 * launches of 4 or 5 columns (for IQ2_XXS, and for every other K-quant and
 * i-quant format but Q6_K and IQ4_NL with K <= 6144 and M >= 4096, from N =
 * 5 on, in 4-column launches).  The results are the narrow kernels' for
 * those N.  Scratch: the tile GEMM uses the context's buffers (see
 * okf_ctx_reserve).  The Q4_K tile GEMM needs them and returns OKF_E_SHAPE
 * where they may not grow (a reserved context that is too small, or a stream
 * being captured into a graph before they were grown); the other formats'
 * tile GEMM then runs without them.  The matvec and narrow paths allocate
 * nothing. */
int okf_gemm(okf_ctx *ctx, const okf_weight *w, const float *X, uint32_t N, float *Y);

/* MetalEnc.gemmTile (MetalEnc.swift:326-352): the tile GEMM for any N >= 1. */
int okf_gemm_tile(okf_ctx *ctx, const okf_weight *w, const float *X, uint32_t N, float *Y);

/* MetalEnc.dequantRow (MetalEnc.swift:402-459): unpack n weights of the row
 * at base + off to fp32, bit-identical to the reference's CPU decoders
 * (GQ.gather, LLM/Gemma/Gemma4Quant.swift:330-364).  row->K, row->M are
 * ignored; n must be a whole number of blocks. */
int okf_dequant_row(okf_ctx *ctx, const okf_weight *row, uint32_t n, float *out);

/* MetalEnc.parallel (MetalEnc.swift:42-47, used for the FFN gate and up
 * projections, LLM/Qwen/QwenMetalEngine.swift:918-923): okf_gemv calls
 * between okf_parallel_begin and okf_parallel_end carry no order among
 * themselves.  They are validated when called and launched at
 * okf_parallel_end, those of one format and one K as a single grid (up to
 * four matrices per launch).  Other calls in the group launch at once.
 * okf_sync inside a group ends it.  Nesting is an OKF_E_ARG. */
int okf_parallel_begin(okf_ctx *ctx);
int okf_parallel_end(okf_ctx *ctx);

/* MetalEnc.addRmsnormBatch (MetalEnc.swift:532-546; kernel add_rmsnorm_batch,
 * LLM/metal/Kernels.metal:2839-2862): for each of `rows` rows of n values,
 * x += r (written back to x), then y = x * w / sqrt(mean(x^2) + eps) with w
 * n fp32 weights.  With r = NULL this is MetalEnc.rmsnormBatch
 * (MetalEnc.swift:516-530, kernel rmsnorm_batch): x is only read.  All
 * pointers are device memory, rows stored contiguously (stride n). */
int okf_add_rmsnorm_batch(okf_ctx *ctx, float *x, const float *r, const float *w, float *y, uint32_t n,
                          uint32_t rows, float eps);

/* MetalEnc.argmaxRows (MetalEnc.swift:496-503; kernel argmax_rows,
 * LLM/metal/Kernels.metal:2756-2795): out[row] = index of the largest of the
 * row's n values, ties to the lower index; NaN never wins and a row with no
 * value above -inf gives 0.  x and out are device memory; rows <= 65535. */
int okf_argmax_rows(okf_ctx *ctx, const float *x, uint32_t n, uint32_t rows, int32_t *out);

/* okf_argmax_rows for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  It has no
 * counterpart in the reference.  Its scratch is a fixed array in device
 * memory, one per GPU, held until the process ends: at most
 * OKF_NOALLOC_ARGMAX_PAIRS (value, index) pairs, i.e. rows * ceil(n / 1024)
 * <= 131072, and rows <= OKF_NOALLOC_ARGMAX_ROWS; larger calls return
 * OKF_E_SHAPE.  It calls no hipMalloc / hipFree and no allocating routine.
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (two streams, two contexts) race. */
#define OKF_NOALLOC_ARGMAX_PAIRS 131072
#define OKF_NOALLOC_ARGMAX_ROWS 4096
int okf_argmax_rows_noalloc(okf_ctx *ctx, const float *x, uint32_t n, uint32_t rows, int32_t *out);

/* A plain streaming read of bytes (a multiple of 16) at the 16-byte-aligned
 * device address p: *out ^= the xor of all its 32-bit words.  No counterpart
 * in the reference: it measures the attainable single-launch HBM read rate
 * that the matvec kernels are compared with (bench.py's hbm_read rows). */
int okf_stream_read(okf_ctx *ctx, const void *p, uint64_t bytes, uint32_t *out);

/* MetalEnc.embedBatch (MetalEnc.swift:1096-1146; kernels embed_batch,
 * q4_k_embed_batch, iq_embed_batch, LLM/metal/Kernels.metal:1444-1482):
 * out[n][K] = row ids[n] of w dequantized to fp32, n < N, bit-identical to
 * okf_dequant_row of that row.  ids is device memory; an id outside
 * [0, M) is clamped to the nearest row. */
int okf_embed_batch(okf_ctx *ctx, const okf_weight *w, const int32_t *ids, uint32_t N, float *out);

/* Waits for all work on the context's stream: the analogue of
 * commit + waitUntilCompleted (LLM/Base/MetalGates.swift:144-149).  Returns
 * OKF_E_HIP if a kernel failed. */
int okf_sync(okf_ctx *ctx);

/* GPUGate.simulate(faultRate:seed:) analogue (MetalGates.swift:101-108):
 * each later launch call fails with OKF_E_INJECTED with probability rate,
 * from a seeded generator, before anything is enqueued.  rate = 0 disables. */
int okf_set_fault_rate(okf_ctx *ctx, double rate, uint64_t seed);

/* The last hipError_t seen by the context (0 if none). */
int okf_last_hip_error(okf_ctx *ctx);

/* Static text for a status code. */
const char *okf_strerror(int status);

/* ---------------------------------------------------------------- GGUF --
 * The weight source: GGUF(path:) (LLM/Base/GGUF.swift:99-151) maps a file and
 * parses its metadata and tensor directory; MetalContext's weight windows
 * (LLM/Base/MetalContext.swift:58-185) make the tensor data GPU-resident.
 * Here okf_gguf_open maps and parses (host only), okf_gguf_upload copies the
 * data region to device memory once, and a tensor's okf_weight is
 * {device base, tensor offset, K = dims[0], M = dims[1] * dims[2] * dims[3],
 * ggml_type}. */
typedef struct okf_gguf okf_gguf;

typedef struct {
    const char *name;    /* NUL-terminated, valid while the file is open */
    uint32_t n_dims;
    uint64_t dims[4];    /* ggml order: dims[0] varies fastest; unused = 1 */
    int32_t ggml_type;
    uint64_t offset;     /* byte offset in the data region */
    uint64_t bytes;      /* GGUF.rowByteCount(type, all elements) */
} okf_gguf_tensor;

int okf_gguf_open(const char *path, okf_gguf **out);
int okf_gguf_close(okf_gguf *g);
int okf_gguf_tensor_count(const okf_gguf *g, uint64_t *n);
int okf_gguf_tensor_at(const okf_gguf *g, uint64_t i, okf_gguf_tensor *t);
/* GGUF.tensor / GGUF.maybe (GGUF.swift:305-311): OKF_E_NOTFOUND if absent */
int okf_gguf_find(const okf_gguf *g, const char *name, okf_gguf_tensor *t);
/* GGUF.int (a bool reads as 0 / 1, GGUF.swift:193-214) */
int okf_gguf_kv_int(const okf_gguf *g, const char *key, int64_t *v);
/* GGUF.double (an int reads as its value) */
int okf_gguf_kv_double(const okf_gguf *g, const char *key, double *v);
/* GGUF.string: pointer and length, valid while the file is open */
int okf_gguf_kv_string(const okf_gguf *g, const char *key, const char **s, uint64_t *len);
/* the mapped data region (host memory) */
int okf_gguf_data(const okf_gguf *g, const void **host, uint64_t *bytes);
/* a device copy of the data region (hipMalloc + copy, synchronous) */
int okf_gguf_upload(okf_ctx *ctx, const okf_gguf *g, void **device);
/* frees a device copy made by okf_gguf_upload */
int okf_gguf_free_device(okf_ctx *ctx, void *device);

#ifdef __cplusplus
}
#endif
#endif
