/*
 * CPU oracle for the quantized-weight matmul path: TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker or the timed CPU baseline.  The product
 * (libkadan_amd.so) never links or calls it.
 *
 * Every function restates, in plain C, the arithmetic of one reference function
 * (cited per declaration; IW = services/hikari/inference_worker, G =
 * IW/third_party/ggml).  Built with -ffp-contract=off so that separately rounded
 * products stay separately rounded, as the reference requires.
 *
 * Pinning (how each function is checked against something other than itself):
 *   kdo_half_to_float      exhaustive 65536 patterns vs the compiled reference
 *                          (oracle/_ref) and vs closed forms (tests/test_oracle.py)
 *   kdo_dequantize_row     reference literal blocks (IW/tests/gguf_quantization.cpp:36-79),
 *                          2048 xorshift blocks/format vs ggml to_float (_ref + fixtures)
 *   kdo_mxfp4_*            E2M1 golden table, 2x64 fixture, extremes and the 2x32
 *                          matvec known answer of IW/tests/quantization.cpp:97-351,
 *                          plus the compiled reference (_ref)
 *   kdo_quantize_*         ggml x86 quantize_row_q8_0 / quantize_row_q8_K (_ref + fixtures),
 *                          and round-half-even ties constructed by hand
 *   kdo_vec_dot_*          ggml AVX2 vec_dot (_ref, fp tolerance) and integer closed forms
 *   kdo_gemv / kdo_gemm_q4_0_q8  brute-force double products over decoded weights,
 *                          linearity and permutation properties
 *   kdo_moe_route/permute  hand-derived cases (2 tokens x 4 experts) and invariants
 *   kdo_moe_gguf_forward   the compiled reference's MoeLayer needs the model runtime,
 *                          so the whole is pinned by a closed-form known answer with the
 *                          sigmoid-gated shared expert (tests/util.py
 *                          known_answer_moe_gguf, float64, no oracle code) and a float64
 *                          numpy composition; its parts individually (decode, products,
 *                          routing)
 *   kdo_moe_forward_f32    not a checker: the timed AVX2 fp32 CPU baseline, checked
 *                          against kdo_moe_forward to fp32 rounding
 *   kdo_moe_forward        the reference never runs MXFP4 weights through MoeLayer
 *                          (IW/src/models/text/qwen_layers.cpp:378-492), so no
 *                          reference output exists for the whole; it is pinned by a
 *                          closed-form known answer worked out from that definition
 *                          (tests/util.py known_answer_moe, float64, no oracle code:
 *                          a dropped silu, swapped gate/up, transposed down or misplaced
 *                          routing weight each fail it) and its parts individually as
 *                          listed above.
 */
#ifndef KADAN_ORACLE_H
#define KADAN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids, as IW/include/kadan/gguf_quantization.hpp:30-55 maps them. */
enum {
    KDO_F32 = 0,
    KDO_F16 = 1,
    KDO_Q4_0 = 2,
    KDO_Q8_0 = 8,
    KDO_Q3_K = 11,
    KDO_Q4_K = 12,
    KDO_Q6_K = 14,
    KDO_IQ3_XXS = 18,
    KDO_IQ4_NL = 20,
    KDO_IQ3_S = 21,
    KDO_IQ2_S = 22,
    KDO_IQ4_XS = 23,
    KDO_BF16 = 30
};

/* IW/include/kadan/gguf_quantization.hpp:576-593: exact IEEE binary16 -> binary32. */
float kdo_half_to_float(uint16_t bits);
/* binary32 -> binary16, round to nearest even (F16C semantics, used for Q8_0 d). */
uint16_t kdo_float_to_half(float value);
/* bfloat16 bits -> binary32 (exact). */
float kdo_bf16_to_float(uint16_t bits);
/* binary32 -> bfloat16 bits, round to nearest even (NaN stays NaN). */
uint16_t kdo_float_to_bf16(float value);

/* IW/include/kadan/gguf_quantization.hpp:65-95 (+ Q4_0: G/src/ggml-common.h block_q4_0). */
int kdo_block_values(int encoding);
int kdo_block_bytes(int encoding);

/* One packed row of `in` values -> fp32, bit-exact to the reference decode:
 * Q8_0    IW/include/kadan/gguf_quantization.hpp:637-641
 * Q4_K    IW/include/kadan/gguf_quantization.hpp:749-761
 * Q3_K    IW/include/kadan/gguf_quantization.hpp:642-657 (G/src/ggml-quants.c:1306, dequantize_row_q3_K)
 * Q6_K    IW/include/kadan/gguf_quantization.hpp:658-673 (G/src/ggml-quants.c:1940, dequantize_row_q6_K)
 * IQ4_NL  IW/include/kadan/gguf_quantization.hpp:695-701 (G/src/ggml-quants.c:2726, dequantize_row_iq4_nl)
 * IQ4_XS  IW/include/kadan/gguf_quantization.hpp:736-748 (G/src/ggml-quants.c:2744, dequantize_row_iq4_xs)
 * BF16    IW/include/kadan/gguf_quantization.hpp:633-636 (one value per 2-byte block)
 * F32, F16 plain values (one per 4- / 2-byte block; F16 through kdo_half_to_float)
 * IQ3_XXS IW/include/kadan/gguf_quantization.hpp:674-694 (G/src/ggml-quants.c dequantize_row_iq3_xxs)
 * IQ2_S   IW/include/kadan/gguf_quantization.hpp:702-718 (dequantize_row_iq2_s)
 * IQ3_S   IW/include/kadan/gguf_quantization.hpp:719-735 (dequantize_row_iq3_s)
 *         (the three lattice grids: kadan_amd/csrc/iq_grids.inc, ggml's tables re-encoded)
 * Q4_0    G/src/ggml-quants.c:459-476 (dequantize_row_q4_0)
 * Returns 0, or -1 for an unknown encoding / ragged row. */
int kdo_dequantize_row(int encoding, const uint8_t* row, size_t in, float* out);

/* Decode-time product semantics of IW/src/cuda/h3_compute.cu:165-228: exactly
 * decoded weights times fp32 inputs.  Accumulates in double (the exact product
 * sum), so the result is the truth the fp32 device sum is compared against.
 * y[r*stride + c] = sum_k w[c,k] * x[r*in + k] for r < rows, c < out. */
int kdo_gemv(int encoding, const uint8_t* weights, size_t row_bytes, const float* x,
             size_t rows, size_t in, size_t out, float* y, size_t stride);

/* G/src/ggml-cpu/arch/x86/quants.c:302-398 quantize_row_q8_0 (AVX2 branch):
 * d = amax/127 stored as fp16 (RNE); id = 127/amax; code = round-half-even(x*id). */
void kdo_quantize_row_q8_0(const float* x, size_t k, int8_t* qs, uint16_t* d_half);

/* G/src/ggml-quants.c:2769-2806 quantize_row_q8_K_ref (used on x86):
 * iscale = -127/max (signed max), nearest_int, clamp 127, bsums per 16, d = 1/iscale. */
void kdo_quantize_row_q8_K(const float* x, size_t k, int8_t* qs, float* d, int16_t* bsums);

/* The prefill activation quantizer of the Q4_0 GEMM (per-32 int8 with an fp32
 * scale): the x86 quantize_row_q8_0 arithmetic above with the scale kept in fp32.
 * x is fp16 bits.  m rows of k values. */
void kdo_quantize_q8_f16(const uint16_t* x, size_t m, size_t k, int8_t* qs, float* d);

/* Integer dots of the CPU baseline (scalar restatements):
 * G/src/ggml-cpu/quants.c:451-479 (q8_0 x q8_0), :696-770 (q4_K x q8_K),
 * :225-260 (q4_0 x q8_0).  Activation blocks use the layouts of the quantizers above. */
float kdo_vec_dot_q8_0_q8_0(size_t k, const uint8_t* w, const int8_t* xq, const uint16_t* xd);
float kdo_vec_dot_q4_0_q8_0(size_t k, const uint8_t* w, const int8_t* xq, const uint16_t* xd);
float kdo_vec_dot_q4_K_q8_K(size_t k, const uint8_t* w, const int8_t* xq, const float* xd,
                            const int16_t* bsums);

/* CPU baseline of IW/src/models/text/cpu_matvec.cpp:28-66 run on the worker split of
 * IW/src/models/text/gguf_weights.cpp:400-446 (64-output-column units):
 * quantize the activation rows, then one vec_dot per (output, row).  threads >= 1. */
int kdo_cpu_matvec(int encoding, const uint8_t* weights, size_t row_bytes, const float* x,
                   size_t rows, size_t in, size_t out, float* y, int threads);

/* Prefill Q4_0 GEMM semantics (ggml vec_dot_q4_0_q8_0 per (m, n), G/src/ggml-cpu/quants.c:225-260)
 * over the activation codes of kdo_quantize_q8_f16: y[m*n_out + n] =
 * sum_b float(sumi_b) * d_w[n,b] * d_x[m,b], accumulated in double. */
int kdo_gemm_q4_0_q8(const uint8_t* weights, size_t n_out, size_t k, const int8_t* xq,
                     const float* xd, size_t m, float* y);

/* IW/src/weights/quantization.cpp:102-110 (E2M1 code -> value). */
float kdo_e2m1(uint8_t code);

/* MXFP4 GPT-OSS layout decode, IW/src/weights/quantization.cpp:79-99,193-205:
 * code of column c in row r = (blocks[r*cols/2 + c/2] >> 4*(c%2)) & 15,
 * w = ldexp(e2m1(code), scales[r*cols/32 + c/32] - 127) computed in double.
 * Returns 0, -1 on shape (cols % 32), -2 on scale 255, -3 on a non-finite value. */
int kdo_mxfp4_decode_rows(const uint8_t* blocks, const uint8_t* scales, size_t rows,
                          size_t cols, float* out);

/* IW/src/weights/quantization.cpp:207-247 matvec: double accumulation, fp32 output.
 * Returns 0, negative on invalid scales / non-finite inputs or results. */
int kdo_mxfp4_matvec(const uint8_t* blocks, const uint8_t* scales, size_t rows, size_t cols,
                     const float* x, float* y);

/* Router of IW/src/models/text/qwen_layers.cpp:403-425: float exp of (l - max), double
 * total, p = float(p/total); the first k of libstdc++'s std::partial_sort of 0..E-1 by
 * p[a] > p[b] (heap select + sort_heap, so equal probabilities come out in the heap's
 * order, :409-416); w_i = p_i / max(sum_i p_i, 6.103515625e-5f).
 * idx, w: [tokens * top_k]. */
void kdo_moe_route(const float* logits, size_t tokens, size_t experts, size_t top_k,
                   int32_t* idx, float* w);

/* Permutation of IW/src/models/text/qwen_layers.cpp:435-451: for each expert e ascending,
 * its slots (token*top_k + i) ascending.  offsets: [experts + 1], perm: [tokens*top_k]. */
void kdo_moe_permute(const int32_t* idx, size_t tokens, size_t top_k, size_t experts,
                     int32_t* offsets, int32_t* perm);

/* The MXFP4 MoE layer as the composition of the reference pieces:
 * route + permute (above), gate/up with kdo_mxfp4_matvec semantics, h = silu(g)*u in
 * float (IW/src/models/text/gguf_weights.cpp:631-633, qwen_layers.cpp:460-464), down,
 * contribution = down * w, y = selection-order float sum (qwen_layers.cpp:469-490).
 * No shared expert.  x: bf16 bits [tokens*hidden]; logits fp32 [tokens*experts];
 * gate/up blocks [experts, inter, hidden/2], scales [experts, inter, hidden/32];
 * down blocks [experts, hidden, inter/2], scales [experts, hidden, inter/32].
 * Outputs y [tokens*hidden]; idx, w [tokens*top_k]; offsets [experts+1]; perm.
 * threads >= 1 (parallel over experts; each expert's arithmetic is sequential).
 * Returns 0 or a negative error. */
int kdo_moe_forward(const uint16_t* x, const float* logits, size_t tokens, size_t hidden,
                    size_t inter, size_t experts, size_t top_k,
                    const uint8_t* gate_blocks, const uint8_t* gate_scales,
                    const uint8_t* up_blocks, const uint8_t* up_scales,
                    const uint8_t* down_blocks, const uint8_t* down_scales,
                    float* y, int32_t* idx, float* w, int32_t* offsets, int32_t* perm,
                    int threads);

/* The layer with fp32 products vectorised with AVX2 FMA (scalar where the CPU lacks it),
 * parallel over 64-row units: a timed CPU baseline beside kdo_moe_forward's exact double
 * flow, not a checker.  Same routing and combine; y within fp32 rounding of
 * kdo_moe_forward's. */
int kdo_moe_forward_f32(const uint16_t* x, const float* logits, size_t tokens, size_t hidden,
                        size_t inter, size_t experts, size_t top_k,
                        const uint8_t* gate_blocks, const uint8_t* gate_scales,
                        const uint8_t* up_blocks, const uint8_t* up_scales,
                        const uint8_t* down_blocks, const uint8_t* down_scales, float* y,
                        int threads);

/* One GGUF weight tensor (host memory): row-major rows of `row_bytes`; expert stacks
 * hold slices of `expert_bytes`. */
typedef struct kdo_gguf_tensor {
    const uint8_t* weights;
    size_t row_bytes;
    size_t expert_bytes;
    int encoding;
} kdo_gguf_tensor;

typedef struct kdo_moe_gguf_layer {
    size_t hidden, experts, top_k, ff, shared_ff;
    kdo_gguf_tensor router, gate_exps, up_exps, down_exps, gate_shexp, up_shexp, down_shexp;
    const float* shared_gate; /* hidden floats */
} kdo_moe_gguf_layer;

/* MoeLayer::forward (IW/src/models/text/qwen_layers.cpp:378-492) over GGUF weights:
 * every projection is kdo_gemv (exactly decoded weights, double-accumulated products,
 * rounded to fp32 once), routing is kdo_moe_route, silu / sigmoid are the reference's
 * fp32 x / (1 + exp(-x)) and 1 / (1 + exp(-x)) (IW/src/models/text/gguf_weights.cpp:
 * 627-633), the shared gate is the reference's sequential fp32 dot, and the
 * contributions are summed in selection order.  y [rows x hidden], idx / w [rows x
 * top_k].  Returns 0, or -1 for a bad argument, -2 when out of memory. */
int kdo_moe_gguf_forward(const kdo_moe_gguf_layer* layer, const float* x, size_t rows,
                         float* y, int32_t* idx, float* w);

#ifdef __cplusplus
}
#endif
#endif
