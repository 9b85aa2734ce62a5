/*
 * moe_oracle.h -- CPU restatement of the com.microsoft MoE / QMoE contrib ops.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links this file;
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it,
 * and only as the checker.
 *
 * Semantics follow the stock ONNX Runtime 1.26 CPU EP, which the reference
 * (MooreThreads/onnxruntime-musa) names as its oracle for every op
 * (test/ops/op_test_utils.py:191-209 builds the CPU session, :274-308 compares
 * with assert_allclose).  The CPU EP sources (contrib_ops/cpu/moe/moe_cpu.cc,
 * contrib_ops/cpu/quantization/moe_quantization_cpu.cc, moe_helper.h) are a
 * third-party dependency pinned at onnxruntime 1.26.0 by the reference's
 * requirements.txt:3 and third_party/README.md:5-6, and are absent from the
 * reference tree; the algorithm restated here is the published one:
 *
 *   router:   p = softmax(logits) (or sigmoid), top-k on the logits with ties
 *             broken toward the lower expert id (reference tie rule,
 *             musa/ep/src/kernels/math/topk_impl.mu:46-65), optional
 *             renormalisation of the k selected probabilities;
 *   dispatch: tokens grouped expert-major, ascending token id within an expert;
 *   experts:  y = fc2(act(fc1(x) [, fc3(x)])) with fp32 accumulation
 *             (fp16/bf16 inputs are widened to fp32, like the reference's
 *             GEMMs computing in fp32, shared_inc/blas_utils.h:187-235);
 *   dequant:  int8 w = (q - 128) * s,  int4 w = (nibble - 8) * s with the
 *             even-k element in the low nibble; s per output channel or per
 *             block of block_size along K;
 *   finalize: out[t] = sum_j w[t,j] * y_{e_j}(x_t), rounded once to T.
 *
 * Parity pins for each function are listed in the oracle section of
 * tests/test_oracle.py.
 */
#ifndef MOE_ORACLE_H_
#define MOE_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types: ONNX TensorProto numbering, as the reference's
 * MusaElementType (musa/ep/src/kernels/shared_inc/device_kernel_types.h:47-62). */
enum { ORC_F32 = 1, ORC_U8 = 2, ORC_F16 = 10, ORC_BF16 = 16 };

/* Activation ids: same numbering as the product header. */
enum { ORC_ACT_RELU = 0, ORC_ACT_GELU = 1, ORC_ACT_SILU = 2, ORC_ACT_IDENTITY = 3,
       ORC_ACT_SWIGLU = 4 };

typedef struct {
  int64_t num_tokens, hidden, inter, num_experts, k;
  int32_t activation;         /* ORC_ACT_* */
  int32_t normalize;          /* normalize_routing_weights */
  int32_t swiglu_fusion;      /* 0 unfused (fc3 = linear), 1 interleaved, 2 chunked */
  float swiglu_limit;         /* +inf when the attribute is absent */
  float alpha, beta;          /* activation_alpha / activation_beta */
  int32_t router_sigmoid;     /* 0 softmax, 1 sigmoid */
  int32_t quant_bits;         /* 0 = float MoE, 4 or 8 = QMoE */
  int64_t block_size;         /* 0 = per output channel */
  int32_t act_dtype;          /* T  : ORC_F32 / ORC_F16 / ORC_BF16 */
  int32_t scale_dtype;        /* T2 : ORC_F32 / ORC_F16 / ORC_BF16 */
  const void *x, *logits;
  const void *w1, *s1, *b1;   /* fc1: [E, f*I, H(/pack)], scales, bias [E, f*I] */
  const void *w2, *s2, *b2;   /* fc2: [E, H, I(/pack)],   scales, bias [E, H] */
  const void *w3, *s3, *b3;   /* fc3 (optional): [E, I, H(/pack)] ... */
  void *out;                  /* [T, H] in act_dtype */
  /* optional diagnostics (may be NULL) */
  int32_t *topk_ids;          /* [T, k] */
  float *topk_w;              /* [T, k] */
  int32_t *expert_offsets;    /* [E + 1] */
  int32_t *perm;              /* [T * k] row -> flat (t*k + j) */
  float *out_f32;             /* [T, H] fp32 result before rounding to T */
  const uint8_t *token_mask;  /* [T]; if set, only tokens with mask != 0 are computed */
  int32_t num_threads;        /* <= 0: OpenMP default */
  int32_t weight_format;      /* 0: integer, zero point 128 / 8 (QMoE); 1: MXFP4 (quant_bits 4,
                                 block_size 32, scales uint8 E8M0) */
} orc_moe_args;

/* Full forward.  Returns 0 on success, nonzero on a bad argument. */
int orc_moe_forward(const orc_moe_args *a);

/* Router only: fp32 logits [T, E] -> ids/weights [T, k]. */
int orc_route(const float *logits, int64_t T, int64_t E, int64_t k, int32_t normalize,
              int32_t sigmoid, int32_t *ids, float *w);

/* Dispatch only: ids [T, k] -> offsets [E+1], perm [T*k] (expert-major, stable). */
int orc_dispatch(const int32_t *ids, int64_t T, int64_t k, int64_t E, int32_t *offsets,
                 int32_t *perm);

/* Dequantize one expert matrix [N, K] to fp32. */
int orc_dequant(const uint8_t *q, const void *scales, int32_t scale_dtype, int32_t bits,
                int64_t block_size, int64_t N, int64_t K, float *out);

/* MXFP4 (OCP Microscaling Formats v1.0: FP4 E2M1 elements, two per byte,
 * even k in the low nibble; one E8M0 scale byte per 32 elements along K):
 * w = e2m1(nibble) * 2^(scale - 127), scale 0xFF = NaN.  [N, K] to fp32. */
int orc_dequant_mxfp4(const uint8_t *q, const uint8_t *scales, int64_t N, int64_t K, float *out);
float orc_e2m1_to_f32(uint32_t nibble);
float orc_e8m0_to_f32(uint32_t e);

/* Activation on one fc1 row (fp32), writing I values.  For fused SwiGLU h1 has
 * 2I entries; for fc3 gating h3 holds the linear half. */
void orc_activation(const float *h1, const float *h3, int64_t I, int32_t activation,
                    int32_t fusion, float alpha, float beta, float limit, float *a);

/* Scalar conversions (RNE), exported for the tests. */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);

#ifdef __cplusplus
}
#endif
#endif /* MOE_ORACLE_H_ */
