/*
 * kadan_amd: MI355X (gfx950) quantized-weight matmul path -- the C ABI.
 *
 * This is the drop-in boundary below the reference worker's C++ projection
 * interface kadan::DenseCompute (IW/include/kadan/dense_compute.hpp:60-342,
 * IW = services/hikari/inference_worker).  Every entry point takes plain device
 * pointers, sizes and a hipStream_t passed as void*; no C++ or torch type crosses
 * it.  All pointers are device pointers unless stated otherwise.  Calls enqueue on
 * `stream` and return without synchronizing (one exception, stated at kdq_moe_gguf: a
 * prefill call over weights nobody has range-checked reads one flag back to the host);
 * a status code other than KDQ_OK means nothing was enqueued (argument errors are
 * detected before any launch).
 *
 * Encodings are named by their GGML type id, as IW/include/kadan/gguf_quantization.hpp:30-55
 * maps them (Q4_0 = 2 is added here; the reference has no kadan encoding for it).
 */
#ifndef KADAN_AMD_H
#define KADAN_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes.  The reference reports these conditions as exception strings
 * (IW/src/cuda/h3_compute.cu:34-37,1767-1830,2178,4047); the host C++ layer
 * (kadan_amd/csrc/hip_dense_compute.cpp) maps each code back to such a string. */
enum kdq_status {
    KDQ_OK = 0,
    KDQ_ERR_ARGUMENT = 1,     /* null pointer, zero or overflowing size */
    KDQ_ERR_SHAPE = 2,        /* "h3_cuda_projection_shape" */
    KDQ_ERR_UNSUPPORTED = 3,  /* encoding/shape outside this implementation */
    KDQ_ERR_ALIAS = 4,        /* "h3_cuda_alias": output overlaps an input */
    KDQ_ERR_HIP = 5,          /* a HIP runtime call failed */
    KDQ_ERR_SCRATCH = 6,      /* "h3_cuda_projection_scratch": workspace allocation */
    KDQ_ERR_ALIGNMENT = 7     /* device pointer alignment the kernels need */
};

/* ---- encodings (GGML type ids; IW/include/kadan/gguf_quantization.hpp:16-55).
 * Every one decodes (kdq_dequantize) and multiplies (kdq_gemv, kdq_gemv_exact,
 * kdq_gemv_batch); Q4_0, Q8_0 and Q4_K also run the streaming / MFMA products and
 * have the tile-packed layout; Q6_K runs the MFMA product (row-major or packed), IQ4_XS,
 * IQ4_NL and Q3_K the MFMA product over their row-major bytes.  Q4_0 is not a kadan device encoding: it is ggml's
 * block_q4_0, added for the prefill GEMM and the products. */
enum kdq_encoding {
    KDQ_F32 = 0,  /* plain fp32 / fp16 matrices (e.g. GGUF routers): exact product only */
    KDQ_F16 = 1,
    KDQ_Q4_0 = 2,
    KDQ_Q8_0 = 8,
    KDQ_Q3_K = 11,
    KDQ_Q4_K = 12,
    KDQ_Q6_K = 14,
    KDQ_IQ3_XXS = 18,
    KDQ_IQ4_NL = 20,
    KDQ_IQ3_S = 21,
    KDQ_IQ2_S = 22,
    KDQ_IQ4_XS = 23,
    KDQ_BF16 = 30
};

/* Human-readable name of a status code (static storage). */
const char* kdq_status_string(int status);

/* Last HIP error text recorded on this thread by a KDQ_ERR_HIP return. */
const char* kdq_last_hip_error(void);

/* Values and bytes per packed block: IW/include/kadan/gguf_quantization.hpp:65-95
 * (gguf::block_values / block_bytes); 0 for an unknown encoding. */
size_t kdq_block_values(int encoding);
size_t kdq_block_bytes(int encoding);

/* Bytes of one packed row of `in` values: IW/include/kadan/device_placement.hpp:115-124
 * (gguf_projection_row_bytes).  0 when `in` is not a whole number of blocks. */
size_t kdq_row_bytes(int encoding, size_t in);

/* ---- prefill decode (replaces gguf_decode_kernel, IW/src/cuda/h3_compute.cu:76-95)
 * Decodes `rows` packed rows of `in` values to fp32 [rows x in], bit-exact to
 * kadan::gguf::decode (IW/include/kadan/gguf_quantization.hpp:631-762) and, for Q4_0,
 * to ggml dequantize_row_q4_0.  When `status` is non-null, *status |= 1 if any decoded
 * value is not finite (the caller zeroes it). */
int kdq_dequantize(int encoding, const void* packed, size_t row_bytes, size_t rows, size_t in,
                   float* out, unsigned* status, void* stream);

/* ---- decode-time product (replaces gguf_matvec_kernel / launch_matvec(const MatvecJob&),
 * IW/src/cuda/h3_compute.cu:165-240,294-306)
 * y[r*stride + c] = sum_k decode(W[c, k]) * x[r*in + k] for r < rows, c < out.
 * W: `out` packed rows of `row_bytes` each.  x: fp32 [rows x in], y: fp32.
 * rows: 1..4096 (more than one pass when needed; gguf_batch_max_rows,
 * IW/include/kadan/dense_compute.hpp:201).  fp32 accumulation.  Q4_0 / Q8_0 / Q4_K
 * (in % 256 == 0, 4-byte aligned rows), Q6_K (in % 256 == 0, 2-byte aligned rows),
 * IQ4_XS (8-byte aligned rows), IQ4_NL (4-byte aligned rows) and Q3_K (2-byte aligned
 * rows):
 * the activation operand is carried as 16-bit
 * block fixed point per 32 values (relative error below 2^-15 of the block maximum),
 * products exact in int32; every other shape and encoding runs kdq_gemv_exact.
 * `status`: as kdq_dequantize, set when a block scale is not finite. */
int kdq_gemv(int encoding, const void* weights, size_t row_bytes, const float* x, size_t rows,
             size_t in, size_t out, float* y, size_t stride, unsigned* status, void* stream);

/* The exact-decode reference kernel: every weight decoded as kdq_dequantize does and
 * multiplied into an fp32 fused multiply-add chain, one wavefront per output.  Any
 * `in` that is a whole number of blocks and a multiple of 8.  The product of the
 * encodings without a streaming kernel, and the cross-check of the others. */
int kdq_gemv_exact(int encoding, const void* weights, size_t row_bytes, const float* x,
                   size_t rows, size_t in, size_t out, float* y, size_t stride,
                   unsigned* status, void* stream);

/* One job of a decode submission: the fields of MatvecJob (IW/src/cuda/h3_compute.cu:110-121)
 * that a caller sets.  All pointers are device pointers. */
typedef struct kdq_matvec_job {
    const void* weights;  /* `columns` packed rows */
    const float* input;   /* rows x in */
    float* output;        /* output[r*stride + c] */
    unsigned* status;     /* optional nonfinite flag */
    size_t row_bytes, stride;
    uint32_t in, columns, rows;
    int32_t encoding;
} kdq_matvec_job;

/* Every job in one submission (replaces launch_matvec(vector<MatvecJob>&, table),
 * IW/src/cuda/h3_compute.cu:367-382, as used by dense_gguf_batch :3963-4375).
 * `jobs` is a HOST array.  Jobs of one shape (encoding, rows in {1, 2, 4, 8}, in) that
 * the streaming kernel takes run together, up to 8 per launch, as the reference runs a
 * submission in one launch per format (h3_compute.cu:336-382); results are bit-identical
 * to one kdq_gemv per job. */
int kdq_gemv_batch(const kdq_matvec_job* jobs, size_t count, void* stream);

/* ---- resident GGUF weights in the tile-packed layout.  No reference counterpart as a
 * format: the reference's device weight bank keeps uploaded packed rows byte for byte
 * (IW/src/cuda/h3_compute.cu:2065-2073,4090-4095); this library's bank (and any caller
 * that keeps weights resident) reorders them once so every wavefront load of the
 * product is whole 128-byte lines.  The bytes are the same bytes, reordered: tiles of
 * 16 rows (zero rows after the last), per tile and 256-value group one unit of
 * 16 x group bytes (Q4_K 2304, Q4_0 2304, Q8_0 4352, Q6_K 3360) of 1 KB code pieces
 * (lane l = 16*chunk + row%16 at 16*l) followed by the block headers / scales (Q6_K's
 * high-bit pairs regrouped per lane within the unit).
 *
 * Device bytes of the packed form of `out` rows of `in` values (0 unless in % 256 == 0). */
size_t kdq_gguf_packed_bytes(int encoding, size_t in, size_t out);

/* Packs `out` rows (`row_bytes` apart, any alignment) into `packed` (16-byte aligned,
 * kdq_gguf_packed_bytes). */
int kdq_gguf_pack(int encoding, const void* weights, size_t row_bytes, size_t in, size_t out,
                  void* packed, void* stream);

/* kdq_gemv over packed weights (replaces gguf_matvec_kernel over resident weights,
 * IW/src/cuda/h3_compute.cu:165-240): same arguments without row_bytes, same results
 * bit for bit as kdq_gemv on the row-major bytes when kdq_gemv runs its MFMA kernel
 * (in % 256 == 0 and in up to ~32K values; larger `in` is KDQ_ERR_UNSUPPORTED here). */
int kdq_gemv_packed(int encoding, const void* packed, const float* x, size_t rows, size_t in,
                    size_t out, float* y, size_t stride, unsigned* status, void* stream);

/* kdq_gemv_batch over packed weights (every job's `weights` packed; `row_bytes` is
 * ignored).  Counterpart of launch_matvec over a submission, h3_compute.cu:367-382. */
int kdq_gemv_packed_batch(const kdq_matvec_job* jobs, size_t count, void* stream);

/* 1 when kdq_gemv_packed takes rows of `in` values of this encoding (a packed form
 * exists and the staged activations fit the kernel's LDS), else 0.  Lets a weight bank
 * choose the resident layout before packing (the reference's gguf_batch_supported,
 * IW/include/kadan/gguf_batch_partition.hpp:15-37, plays this role for its bank). */
int kdq_gemv_packed_supported(int encoding, size_t in);

/* ---- prefill Q4_0 GEMM (no reference device counterpart; the reference decodes to
 * F32 and calls cublasSgemm, IW/src/cuda/h3_compute.cu:2451, and its CPU path runs
 * ggml vec_dot_q4_0_q8_0, G/src/ggml-cpu/quants.c:225-260).
 * Activations: fp16 [m x k] quantized per 32 to int8 with an fp32 scale
 * (amax/127, codes round-half-even(x*127/amax), G/src/ggml-cpu/arch/x86/quants.c:302-398).
 * y[m x n] fp16 = sum_b float(sumi_b) * d_w * d_x, fp32 accumulation.
 * k % 256 == 0; any m, n >= 1. */
int kdq_gemm_q4_0(const void* weights, size_t n, size_t k, const uint16_t* x_f16, size_t m,
                  uint16_t* y_f16, void* stream);

/* kdq_gemm_q4_0 over the tile-packed Q4_0 layout of kdq_gguf_pack (the resident form
 * the decode product kdq_gemv_packed reads, so one resident copy serves decode and
 * prefill): `packed` holds kdq_gguf_packed_bytes(KDQ_Q4_0, k, n) bytes, 16-byte
 * aligned.  Same semantics as kdq_gemm_q4_0 (same activation quantisation, fp16
 * products of fp16(code * d_x) and fp16((q - 8) * d_w), fp32 accumulation); results
 * may differ from kdq_gemm_q4_0 in the last fp32 bits (summation order). */
int kdq_gemm_q4_0_packed(const void* packed, size_t n, size_t k, const uint16_t* x_f16,
                         size_t m, uint16_t* y_f16, void* stream);

/* ---- prefill GEMM for the kadan encodings over the tile-packed bank copy (replaces the
 * decode-to-F32 tile + cublasSgemm of project<float>, IW/src/cuda/h3_compute.cu:2201-2218,
 * 2451, behind dense_gguf_source with more than gguf_batch_rows input rows).
 * y[m x n] fp32 = x[m x k] fp32 . W^T, W = `n` rows of `k` values of Q4_K, Q8_0 or Q6_K
 * in the tile-packed layout (kdq_gguf_pack: kdq_gguf_packed_bytes(encoding, k, n)
 * bytes, 16-byte aligned).  Activations are scaled per row by a power of two and rounded
 * once to fp16; weights are dequantised to fp16 (Q8_0: d * q; Q4_K: q * fp16(d * sc) -
 * fp16(dmin * m); Q6_K: (q - 32) * fp16(d * sc)); products accumulate in fp32.
 * k % 256 == 0, k <= 32768; x 16-byte aligned.  `status` (optional, zeroed by the
 * caller): |= 1 for a non-finite weight scale, |= 2 when a dequantised weight could pass
 * the fp16 range (those outputs are not to be used: run kdq_gemv_packed instead). */
int kdq_gemm_packed(int encoding, const void* packed, size_t n, size_t k, const float* x,
                    size_t m, float* y, unsigned* status, void* stream);

/* ---- prefill GEMM over row-major GGUF rows, any encoding (replaces the same decode-to-
 * F32 tile + cublasSgemm, IW/src/cuda/h3_compute.cu:2201-2218,2451, for the encodings the
 * packed GEMM does not take: Q3_K, IQ4_XS, IQ4_NL, IQ3_XXS, IQ3_S, IQ2_S, BF16, Q4_0; it
 * also runs Q4_K, Q8_0 and Q6_K rows as they lie in the file).
 * y[m x n] fp32 = x[m x k] fp32 . W^T, W = `n` rows of `row_bytes` (>= kdq_row_bytes, even)
 * as the file holds them, 2-byte aligned.  Every weight is decoded exactly as
 * kdq_dequantize does, then rounded once to fp16; activations are scaled per row by a
 * power of two and rounded once to fp16; products accumulate in fp32.  Each workgroup
 * reads the bytes of its 128 weight rows once for 128 activation rows.
 * k % kdq_gemm_rows_values(encoding) == 0 (256; BF16 64), k <= 65536; x and y 16-byte
 * aligned.  `status` (optional, zeroed by the caller): |= 1 for a non-finite decoded
 * weight (for Q4_0, Q8_0, Q4_K, Q3_K, IQ4_NL and IQ4_XS: a non-finite block scale), |= 2
 * for a weight past the fp16 range (for those encodings: a block scale that could take
 * one past it, as kdq_gemm_packed checks) -- then run kdq_gemv for these rows. */
size_t kdq_gemm_rows_values(int encoding);
int kdq_gemm_rows(int encoding, const void* weights, size_t row_bytes, size_t n, size_t k,
                  const float* x, size_t m, float* y, unsigned* status, void* stream);

/* The activation quantizer of kdq_gemm_q4_0 on its own (for bit-exact checks):
 * q int8 [m x k], d fp32 [m x k/32]. */
int kdq_quantize_q8(const uint16_t* x_f16, size_t m, size_t k, int8_t* q, float* d,
                    void* stream);

/* ---- GGUF mixture-of-experts layer (the reference runs it on the host, calling the
 * device three times: MoeLayer::forward, IW/src/models/text/qwen_layers.cpp:378-492;
 * this is one stream-ordered submission with device-side routing).
 * One weight tensor: `weights` (device) holds row-major GGUF rows of `row_bytes`; an
 * expert stack holds `experts` slices of `expert_bytes` each (a multiple of 16). */
typedef struct kdq_gguf_tensor {
    const void* weights;
    size_t row_bytes;
    size_t expert_bytes; /* expert stacks only */
    int32_t encoding;    /* kdq_encoding */
} kdq_gguf_tensor;

/* The layer's MoeSpec (IW/src/models/text/qwen_layers.hpp:96-98) and tensors
 * (bind_moe, qwen_layers.cpp:357-371). */
typedef struct kdq_moe_gguf_layer {
    size_t hidden, experts, top_k, ff, shared_ff;
    kdq_gguf_tensor router;     /* ffn_gate_inp: experts x hidden */
    kdq_gguf_tensor gate_exps;  /* ffn_gate_exps: experts x (ff x hidden) */
    kdq_gguf_tensor up_exps;    /* ffn_up_exps: experts x (ff x hidden) */
    kdq_gguf_tensor down_exps;  /* ffn_down_exps: experts x (hidden x ff) */
    kdq_gguf_tensor gate_shexp; /* ffn_gate_shexp: shared_ff x hidden */
    kdq_gguf_tensor up_shexp;   /* ffn_up_shexp: shared_ff x hidden */
    kdq_gguf_tensor down_shexp; /* ffn_down_shexp: hidden x shared_ff */
    const float* shared_gate;   /* ffn_gate_inp_shexp: hidden floats */
} kdq_moe_gguf_layer;

/* y[rows x hidden] = MoeLayer::forward(x[rows x hidden]) (qwen_layers.cpp:378-492):
 * router softmax (double total), top-k by probability, weights / max(sum, 2^-14); per
 * selection silu(gate_e . x) * (up_e . x) -> down_e, summed in selection order with
 * its weight; plus the shared expert's down(silu(gate_s . x) * (up_s . x)) scaled by
 * sigmoid(shared_gate . x).  Optional outputs: `selected` / `weights` [rows x top_k]
 * (the routing), `status` |= 1 for a non-finite weight scale.  Every projection decodes
 * its weights exactly (kdq_gemv semantics).  rows <= 4096, rows * top_k <= 8192,
 * experts <= 256, top_k <= 8; x, y, shared_gate 16-byte aligned.  Up to 8 rows run
 * every slot's expert product directly; larger batches (prefill chunks) group the
 * slots by expert, either into 8-row items of the decode product (an expert's weights
 * read once per 8 of its rows, the reference's per-expert batch jobs,
 * IW/include/kadan/dense_compute.hpp:197-201) or, for Q4_K / Q8_0 / Q6_K, into 64-row
 * tiles of the prefill GEMM (fp16 operands, fp32 accumulation).
 * Up to 8 rows (rows x hidden x 4 bytes <= 64 KB) with an F32 router and the common
 * K-quant mixes run in two launches whose
 * workgroups hand the routing and the rows to combine to one another through
 * device-wide counters (one set per GPU): calls that overlap on one GPU race (as they
 * do on the library's workspace); `status` |= 8 if a workgroup waited past its bound
 * for the routing (the output is then not the layer's).  The call number those counters
 * compare lives on the device, so the two launches may be captured in a graph and
 * replayed (after one call outside the capture has sized the workspace).
 * Host wait: when the prefill GEMM runs here, this call packs the weights itself and
 * cannot know in advance whether a block scale could take a dequantised weight past
 * the fp16 range (never so in real checkpoints); it copies the GEMM's flag to the host
 * and synchronizes `stream` once, mid-layer, and on that flag redoes the expert
 * products on the exact decode.  Callers that must not block use kdq_moe_gguf_packed
 * with copies checked once by kdq_gguf_gemm_check (`checked` = 1): it never waits. */
int kdq_moe_gguf(const kdq_moe_gguf_layer* layer, const float* x, size_t rows, float* y,
                 int32_t* selected, float* weights, unsigned* status, void* stream);

/* Tile-packed copies of a GGUF MoE layer's matrices that a caller keeps resident (a
 * weight bank): each non-null pointer replaces the packing kdq_moe_gguf does in every
 * prefill call for that matrix.  Expert stacks are packed as one matrix of experts x rows
 * rows: kdq_gguf_pack(encoding, weights, row_bytes, in, experts * rows, out) (gate/up:
 * in = hidden, rows = ff; down: in = ff, rows = hidden); shared matrices as themselves.
 * Only the encodings the prefill GEMM takes (Q4_K, Q8_0, Q6_K) are read packed. */
typedef struct kdq_moe_gguf_packed_stacks {
    const void* gate_exps;
    const void* up_exps;
    const void* down_exps;
    const void* gate_shexp;
    const void* up_shexp;
    const void* down_shexp;
    /* 1 when kdq_gguf_gemm_check found no flag in any matrix given here: the layer then
     * never waits on the host for the prefill GEMM's range flag (see kdq_moe_gguf) */
    unsigned checked;
} kdq_moe_gguf_packed_stacks;

/* The prefill GEMM's scale checks over a tile-packed matrix (n rows of k inputs), once,
 * without the product: *flags (device memory) |= 1 for a non-finite scale, |= 2 when a
 * dequantised weight could pass the fp16 range (the GEMM would then refuse the matrix
 * and its callers take the exact-decode products).  Q4_K, Q8_0, Q6_K.  No counterpart in
 * the reference (it decodes to fp32); for callers that keep packed copies resident. */
int kdq_gguf_gemm_check(int encoding, const void* packed, size_t n, size_t k, unsigned* flags,
                        void* stream);

/* kdq_moe_gguf with resident packed copies (`packed` may be null: kdq_moe_gguf).  No
 * counterpart in the reference, whose layer reads every expert through DenseCompute
 * batch jobs (IW/include/kadan/dense_compute.hpp:197-201); the row-major tensors of
 * `layer` stay required (decode batches and the exact fallback read them) and must hold
 * the same weights as the packed copies.  Same results as kdq_moe_gguf; with
 * `packed->checked` = 1 it returns without synchronizing. */
int kdq_moe_gguf_packed(const kdq_moe_gguf_layer* layer, const kdq_moe_gguf_packed_stacks* packed,
                        const float* x, size_t rows, float* y, int32_t* selected, float* weights,
                        unsigned* status, void* stream);

/* ---- MXFP4 mixture-of-experts layer (the reference has no device MoE; this composes
 * MoeLayer::forward, IW/src/models/text/qwen_layers.cpp:378-492, with the MXFP4
 * product semantics of IW/src/weights/quantization.cpp:79-99,207-247).
 * Weights in the GPT-OSS layout (IW/include/kadan/checkpoint.hpp:151-163):
 *   gate/up blocks u8 [experts, inter, hidden/2], scales u8 [experts, inter, hidden/32]
 *   down    blocks u8 [experts, hidden, inter/2], scales u8 [experts, hidden, inter/32]
 * element 2i = low nibble of byte i; w = e2m1(code) * 2^(scale-127). */

/* Router + top-k + permutation, IW/src/models/text/qwen_layers.cpp:403-451.
 * logits fp32 [tokens x experts]; top_k <= 8; experts <= 256.
 * idx int32 [tokens x top_k] (selection order: the first top_k of std::partial_sort by
 * probability descending, equal probabilities in its heap order), w fp32 [tokens x top_k]
 * renormalised weights,
 * offsets int32 [experts + 1], perm int32 [tokens*top_k] = slots (token*top_k + i)
 * grouped by expert ascending, slot ascending within an expert. */
int kdq_moe_route(const float* logits, size_t tokens, size_t experts, size_t top_k,
                  int32_t* idx, float* w, int32_t* offsets, int32_t* perm, void* stream);

/* Decodes MXFP4 rows to fp32 exactly (IW/src/weights/quantization.cpp:193-205):
 * blocks [rows x cols/2], scales [rows x cols/32] -> out [rows x cols].
 * *status |= 1 for a scale byte of 255, |= 2 for a value that overflows fp32. */
int kdq_mxfp4_dequantize(const uint8_t* blocks, const uint8_t* scales, size_t rows,
                         size_t cols, float* out, unsigned* status, void* stream);

/* The whole layer: y fp32 [tokens x hidden] from x bf16 [tokens x hidden] and logits.
 * Also returns the routing (idx, w, offsets, perm as kdq_moe_route) when those
 * pointers are non-null.  hidden % 64 == 0, inter % 64 == 0; x, y and the three block
 * arrays 16-byte aligned.  The weights are repacked (kdq_moe_mxfp4_pack) into the
 * workspace on every call: callers that keep weights resident pack once and call
 * kdq_moe_mxfp4_packed.  Counterpart of MoeLayer::forward (qwen_layers.cpp:378-492). */
int kdq_moe_mxfp4(const uint16_t* x_bf16, const float* logits, size_t tokens, size_t hidden,
                  size_t inter, size_t experts, size_t top_k,
                  const uint8_t* gate_blocks, const uint8_t* gate_scales,
                  const uint8_t* up_blocks, const uint8_t* up_scales,
                  const uint8_t* down_blocks, const uint8_t* down_scales,
                  float* y, int32_t* idx, float* w, int32_t* offsets, int32_t* perm,
                  void* stream);

/* Device bytes of one packed projection tensor of `experts` x [rows x cols] MXFP4 values
 * (0 unless rows % 32 == 0 and cols % 64 == 0).  No reference counterpart: the packed
 * layout is this library's resident weight format (the reference keeps resident GGUF
 * weights in its bank, IW/src/cuda/h3_compute.cu weight cache; MoE weights stay on the
 * host, IW/src/models/text/qwen_layers.cpp:455-489). */
size_t kdq_moe_mxfp4_packed_bytes(size_t experts, size_t rows, size_t cols);

/* Repacks one projection tensor (gate, up: rows = inter, cols = hidden; down: rows =
 * hidden, cols = inter) from the GPT-OSS layout into `packed` (kdq_moe_mxfp4_packed_bytes,
 * 256-byte aligned; blocks 16-byte aligned).  Per expert, per group of 32 rows and step of
 * 64 values, the codes form one 1 KB block (lane i + 32h: bytes 32q + 16h .. +15 of row
 * 32g + i); per 4 steps the scales form one 256-byte block (lane dword byte j: scale of
 * step 4p + j, half h).  Codes and scale bytes are copied unchanged. */
int kdq_moe_mxfp4_pack(const uint8_t* blocks, const uint8_t* scales, size_t experts,
                       size_t rows, size_t cols, uint8_t* packed, void* stream);

/* kdq_moe_mxfp4 over packed weights (each 256-byte aligned). */
int kdq_moe_mxfp4_packed(const uint16_t* x_bf16, const float* logits, size_t tokens,
                         size_t hidden, size_t inter, size_t experts, size_t top_k,
                         const uint8_t* gate_packed, const uint8_t* up_packed,
                         const uint8_t* down_packed, float* y, int32_t* idx, float* w,
                         int32_t* offsets, int32_t* perm, void* stream);

/* kdq_moe_mxfp4_packed without any allocation.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, kernels and results
 * (bit for bit) as kdq_moe_mxfp4_packed; the layer's scratch lives in a static device
 * array of 64 MiB that each device holds for the life of the process, and a layer whose
 * scratch does not fit it is refused with KDQ_ERR_SCRATCH (at the C4 geometry, 32
 * experts of 2880 x 2880: up to 128 tokens; with 128 experts: up to 16 tokens).  It
 * calls no hipMalloc / hipFree.  Every call on a device shares that device's array:
 * calls that overlap on one device (other streams, other threads) race. */
int kdq_moe_mxfp4_packed_noalloc(const uint16_t* x_bf16, const float* logits, size_t tokens,
                                 size_t hidden, size_t inter, size_t experts, size_t top_k,
                                 const uint8_t* gate_packed, const uint8_t* up_packed,
                                 const uint8_t* down_packed, float* y, int32_t* idx,
                                 float* w, int32_t* offsets, int32_t* perm, void* stream);

/* Measurement aid, no counterpart in the reference: one streaming read of `bytes`
 * (a multiple of 16; `src` 16-byte aligned) over `workgroups` workgroups of `threads`
 * (256 or 1024) lanes.  Workgroup b folds (xor) the 32-bit words of its share, units of
 * 16 bytes [b * per, (b + 1) * per) with per = ceil(units / workgroups) rounded up to a
 * multiple of 64, and stores the fold into sink[b] always (store_all != 0) or only when
 * it equals `match`.  Its best time over launch shapes is the HBM read ceiling the
 * GEMV's bandwidth is judged against. */
int kdq_hbm_read(const void* src, size_t bytes, unsigned* sink, size_t workgroups,
                 int threads, int store_all, unsigned match, void* stream);

/* Frees this thread's current device's cached workspace (synchronizes the device).
 * IW/include/kadan/dense_compute.hpp:66-68 release_scratch counterpart. */
int kdq_release_scratch(void);

#ifdef __cplusplus
}
#endif
#endif
