/*
 * tinyinfer_mxfp4.h -- C ABI of the MI355X (gfx950) MXFP4 weight-only MLP.
 *
 * Plain pointers and sizes only. Every pointer is a device pointer on the
 * current HIP device unless stated otherwise. `stream` is a hipStream_t
 * passed as void* (NULL = the legacy default stream). Work is enqueued
 * asynchronously and nothing here synchronizes, except where a function says
 * it does. Every function returns 0 on success or a TI_* status code, and
 * never throws.
 *
 * Threads: every function may be called from any host thread, also
 * concurrently; calls on one stream are ordered by the stream.  The library's
 * shared state (device properties, tuning options, split-K workspaces) is
 * initialised once and guarded.  Split-K workspaces are per (device, stream):
 * graphs captured on one stream share that stream's workspace, so replays of
 * such graphs must not run at the same time as each other, or as calls on
 * the capture stream.
 *
 * Layout (reference tinyinfer/layers/linear.py:36-48,
 * tinyinfer/quantization/quantize_mxfp4.py:233-253):
 *   X           [N, hidden]                    bf16 or fp16, row-major
 *   gate, up    [intermediate, hidden/2]       uint8, e2m1 pairs, low nibble first
 *   gate_scale,
 *   up_scale    [intermediate, hidden/32]      uint8 e8m0 (byte = exponent + 127)
 *   down        [hidden, intermediate/2]       uint8
 *   down_scale  [hidden, intermediate/32]      uint8
 *   tmp         [N, intermediate]              activation dtype (SiLU(g)*u)
 *   O           [N, hidden]                    activation dtype
 */
#ifndef TINYINFER_MXFP4_H_
#define TINYINFER_MXFP4_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define TI_OK 0
#define TI_ERR_INVALID_ARG 1      /* null pointer, zero/negative size, bad enum */
#define TI_ERR_BAD_SHAPE 2        /* hidden or intermediate not a multiple of 32 */
#define TI_ERR_BAD_DTYPE 3        /* dtype code not supported by this entry point */
#define TI_ERR_HIP 4              /* a HIP runtime call failed (see last HIP error) */
#define TI_ERR_NO_DEVICE 5        /* no gfx950 device is current */
#define TI_ERR_TOO_LARGE 6        /* a size exceeds what the kernels index */
#define TI_ERR_MISALIGNED 7       /* X, gate, up, down or tmp not 16-byte aligned */
#define TI_ERR_UNSUPPORTED 8      /* a forced kernel path cannot run this call */
#define TI_ERR_SCRATCH 9          /* the no-alloc entry point's fixed scratch is too small for the call */

/* dtype codes: the reference's dtype_code values (mlp_fp4.cu:481-515), plus fp32. */
#define TI_DTYPE_F16 0
#define TI_DTYPE_BF16 1
#define TI_DTYPE_F32 2

/* Kernel paths for tinyinfer_mlp_forward_mxfp4_path. */
#define TI_PATH_AUTO 0            /* same choice as tinyinfer_mlp_forward_mxfp4 */
#define TI_PATH_SKINNY 1          /* dequant skinny-GEMM on MFMA (weights streamed once per 64 tokens) */
#define TI_PATH_GEMM 2            /* LDS-tiled dequant -> bf16 MFMA GEMM */
#define TI_PATH_DECODE 3          /* fused single-launch decode kernel (N <= 4, full MLP only) */

/* Quantizer flag bits written to *flags by tinyinfer_mxfp4_quantize. */
#define TI_QFLAG_NONFINITE 1u     /* NaN/Inf in the input */
#define TI_QFLAG_EXP_RANGE 2u     /* a block exponent falls outside [-127, 127] */

/*
 * Fused MXFP4 MLP forward: O = down( SiLU(X gate^T) * (X up^T) ).
 * Replaces the reference's C entry point
 *   extern "C" void mlp_forward_mxfp4_cuda(X, gate, gate_scale, up, up_scale,
 *       down, down_scale, N, hidden_dim, intermediate, tmp, O, dtype_code)
 *   (tinyinfer/csrc/mlp_fp4.cu:466-518, declared tinyinfer/csrc/bind.cpp:640-654)
 * with the same arguments in the same order, plus `stream`; errors are
 * returned instead of thrown. `tmp` must hold N*intermediate elements of the
 * activation dtype; on return it holds bf16/fp16 SiLU(g)*u, as in the
 * reference. The kernel path is chosen from N: for N <= 8 the streaming
 * decode kernels (one launch per stage) when hidden and intermediate are
 * multiples of 512 and the shape fits their LDS plan, else the skinny kernels
 * up to N < 96, else the tiled GEMM. X, gate, up, down and tmp must be
 * 16-byte aligned. Calls of the fused decode path (TI_PATH_DECODE) must not
 * overlap on one device (its workgroups synchronise through device memory).
 */
int tinyinfer_mlp_forward_mxfp4(const void* X, const uint8_t* gate, const uint8_t* gate_scale,
                                const uint8_t* up, const uint8_t* up_scale, const uint8_t* down,
                                const uint8_t* down_scale, size_t N, size_t hidden_dim,
                                size_t intermediate, void* tmp, void* O, int dtype_code,
                                void* stream);

/*
 * tinyinfer_mlp_forward_mxfp4 without any device allocation. No counterpart
 * in the reference: it is for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels and results as tinyinfer_mlp_forward_mxfp4; the
 * split-K partial sums go to a fixed 64 MiB device array of the library (one
 * per device, held until the process ends) instead of an allocated
 * workspace, and no hipMalloc/hipFree is called.  A call of up to 64 tokens
 * whose split-K tile kernels would need more than 64 MiB (far beyond the
 * Qwen3 MLP shapes) is refused with TI_ERR_SCRATCH; from 65 tokens such a
 * call runs on the GEMM path instead (kernels, and so bits, may then differ
 * from tinyinfer_mlp_forward_mxfp4's, within the parity bar); the GEMM path
 * splits K only as far as the array holds.  All calls on one device share its array: calls that overlap
 * on a device (other streams or threads, concurrent graph replays) race and
 * must not run at the same time.
 */
int tinyinfer_mlp_forward_mxfp4_noalloc(const void* X, const uint8_t* gate, const uint8_t* gate_scale,
                                        const uint8_t* up, const uint8_t* up_scale, const uint8_t* down,
                                        const uint8_t* down_scale, size_t N, size_t hidden_dim,
                                        size_t intermediate, void* tmp, void* O, int dtype_code,
                                        void* stream);

/*
 * Same as tinyinfer_mlp_forward_mxfp4 with the kernel path forced
 * (TI_PATH_*). No reference counterpart: the reference has one path. Used by
 * parity tests and the benchmark to exercise both kernels at any N.
 */
int tinyinfer_mlp_forward_mxfp4_path(const void* X, const uint8_t* gate, const uint8_t* gate_scale,
                                     const uint8_t* up, const uint8_t* up_scale,
                                     const uint8_t* down, const uint8_t* down_scale, size_t N,
                                     size_t hidden_dim, size_t intermediate, void* tmp, void* O,
                                     int dtype_code, int path, void* stream);

/*
 * The gate_up stage alone: tmp = SiLU(X gate^T) * (X up^T), rounded once to
 * the activation dtype. Replaces the reference's first kernel,
 * mlp_stage1_mxfp4 (tinyinfer/csrc/mlp_fp4.cu:79-142, launched at :457);
 * `path` as in tinyinfer_mlp_forward_mxfp4_path. The down pointers of the
 * full entry point are not taken.
 */
int tinyinfer_mlp_gate_up_mxfp4(const void* X, const uint8_t* gate, const uint8_t* gate_scale,
                                const uint8_t* up, const uint8_t* up_scale, size_t N,
                                size_t hidden_dim, size_t intermediate, void* tmp, int dtype_code,
                                int path, void* stream);

/*
 * The down stage alone: O = tmp down^T, rounded once to the activation dtype.
 * Replaces the reference's second kernel, mlp_stage2_mxfp4
 * (tinyinfer/csrc/mlp_fp4.cu:365-426, launched at :459). `tmp` is
 * [N, intermediate] in the activation dtype.
 */
int tinyinfer_mlp_down_mxfp4(const void* tmp, const uint8_t* down, const uint8_t* down_scale,
                             size_t N, size_t hidden_dim, size_t intermediate, void* O,
                             int dtype_code, int path, void* stream);

/*
 * The MLP followed by the decoder layer's residual add, fused into the down
 * stage's epilogue: O = residual + MLP(X), where MLP(X) is first rounded to
 * the activation dtype and the sum is taken in fp32 and rounded again --
 * bit-identical to tinyinfer_mlp_forward_mxfp4 followed by the reference's
 * `hidden_states = residual + hidden_states` (tinyinfer/models/qwen3.py:219)
 * on two activation-dtype tensors, without that extra launch and [N, hidden]
 * round trip. `residual` is [N, hidden] in the activation dtype, 16-byte
 * aligned; O may be residual itself (in-place). `path` as in
 * tinyinfer_mlp_forward_mxfp4_path.
 */
int tinyinfer_mlp_forward_mxfp4_residual(const void* X, const uint8_t* gate, const uint8_t* gate_scale,
                                         const uint8_t* up, const uint8_t* up_scale,
                                         const uint8_t* down, const uint8_t* down_scale, size_t N,
                                         size_t hidden_dim, size_t intermediate, void* tmp,
                                         const void* residual, void* O, int dtype_code, int path,
                                         void* stream);

/*
 * The decoder layer's MLP half with both neighbours fused
 * (tinyinfer/models/qwen3.py:210-219: residual = hidden; hidden =
 * post_attention_layernorm(hidden); hidden = mlp(hidden); hidden = residual +
 * hidden), for a hidden state X [N, hidden]:
 *   xn = round(norm_weight * X * rsqrt(sum(X^2) / hidden + eps))   per row
 *   O  = round(X + round(MLP(xn)))
 * The RMSNorm is the reference's rmsnorm_forward_cuda
 * (tinyinfer/csrc/rmsnorm.cu:10-54, through layernorm.py:15-23): fp32 inside,
 * (w * x) * inv in that order. `xn` [N, hidden] receives the normalized rows.
 * On the streaming decode kernels (N <= 8, AUTO or TI_PATH_SKINNY) the norm
 * runs in the gate_up kernel's prologue on its LDS copy of X, so the layer
 * half is two launches; on the other paths a norm kernel writes xn first.
 * norm_weight [hidden] and xn are in the activation dtype, 16-byte aligned;
 * O may be X itself (in-place). `path` as in tinyinfer_mlp_forward_mxfp4_path.
 */
int tinyinfer_mlp_forward_mxfp4_rmsnorm(const void* X, const void* norm_weight, float eps,
                                        const uint8_t* gate, const uint8_t* gate_scale, const uint8_t* up,
                                        const uint8_t* up_scale, const uint8_t* down,
                                        const uint8_t* down_scale, size_t N, size_t hidden_dim,
                                        size_t intermediate, void* xn, void* tmp, void* O, int dtype_code,
                                        int path, void* stream);

/*
 * RMSNorm alone, the reference's rmsnorm_forward_cuda
 * (tinyinfer/csrc/rmsnorm.cu:79-123) for fp16 and bf16 rows:
 * O = round(weight * X * rsqrt(sum(X^2) / hidden + eps)) per row of
 * `hidden_dim` activations. hidden_dim a multiple of 8; X, weight and O
 * 16-byte aligned.
 */
int tinyinfer_rmsnorm(const void* X, const void* weight, float eps, size_t num_rows, size_t hidden_dim, void* O,
                      int dtype_code, void* stream);

/*
 * One MXFP4 linear layer on the down stage's kernels: O = X W^T (+ residual
 * when non-null, rounded as above), W [out_features, in_features/2] packed
 * with scales [out_features, in_features/32] in the checkpoint layout. The
 * reference computes its dense linears with F.linear
 * (tinyinfer/layers/linear.py:8-31); this is that call for weights kept in
 * MXFP4 (qkv_proj, o_proj, lm_head), dequantized exactly in the kernel with
 * one rounding of the fp32 sum. in_features and out_features must be
 * multiples of 32; X, W, O (and residual) 16-byte aligned. `path` as in
 * tinyinfer_mlp_forward_mxfp4_path (TI_PATH_DECODE is refused).
 */
int tinyinfer_mxfp4_linear(const void* X, const uint8_t* w, const uint8_t* w_scale, size_t N,
                           size_t in_features, size_t out_features, const void* residual, void* O,
                           int dtype_code, int path, void* stream);

/*
 * Device dequantization: out[rows, k] = e2m1(packed) * 2^(scale-127), bit-exact.
 * Replaces dequantize_chunk (tinyinfer/quantization/quantize_mxfp4.py:67-85)
 * and the device decode helpers decode_e2m1 / decode_e8m0
 * (tinyinfer/csrc/utils.h:87-127). out_dtype is TI_DTYPE_F32 or TI_DTYPE_BF16
 * (every value is exact in both). Scale byte 255 yields NaN, as the reference
 * GPU decode does; the reference CPU decode raises on it instead, and the
 * Python wrapper does the same.
 */
int tinyinfer_mxfp4_dequant(const uint8_t* packed, const uint8_t* scale, size_t rows, size_t k,
                            void* out, int out_dtype, void* stream);

/*
 * Device quantization, bit-exact with the reference quantizer:
 * quantize_chunk (tinyinfer/quantization/quantize_mxfp4.py:28-64).
 * w[rows, k] in TI_DTYPE_F32 / BF16 / F16 -> packed[rows, k/2], scale[rows, k/32].
 * `flags` is a device uint32 that the kernel ORs TI_QFLAG_* bits into; this
 * function clears it first. The caller reads it after the stream completes.
 * Where the reference raises ValueError, the bytes written for the offending
 * blocks are unspecified.
 */
int tinyinfer_mxfp4_quantize(const void* w, int in_dtype, size_t rows, size_t k, uint8_t* packed,
                             uint8_t* scale, uint32_t* flags, void* stream);

/*
 * Diagnostics of the current device (synchronous): the number of times the
 * fused decode kernel's wait for the other workgroups gave up since the
 * library was loaded or tinyinfer_mxfp4_decode_reset last ran (a safety bound
 * that only trips if its workgroups were not all resident).  The result of
 * the call that timed out is invalid, and while the count is nonzero every
 * later TI_PATH_DECODE call returns TI_OK but leaves tmp and O unwritten (its
 * kernel exits at entry). No reference counterpart.
 */
int tinyinfer_mxfp4_diagnostics(uint32_t* decode_barrier_timeouts);

/*
 * Synchronizes the current device and clears the fused decode kernel's
 * cross-workgroup state (flags, epoch, the poison left by a timed-out wait,
 * the timeout count). No reference counterpart.
 */
int tinyinfer_mxfp4_decode_reset(void);

/*
 * Tuning options, by the name of the environment variable that sets each at
 * load (TINYINFER_ROWSTREAM, TINYINFER_ROWPAIR, TINYINFER_TILE,
 * TINYINFER_TILE_GU, TINYINFER_ROW_SPLIT_GATEUP, TINYINFER_ROW_SPLIT_DOWN,
 * TINYINFER_GEMM_RING, TINYINFER_RING_KSPLIT, TINYINFER_RING_TAIL,
 * TINYINFER_RING_WR_GU / _DN,
 * TINYINFER_RING_NW_GU / _DN, TINYINFER_SKINNY_NW, TINYINFER_STREAM_SPU_GU /
 * _DN, TINYINFER_STREAM_XREG, TINYINFER_WORKSPACE_MB, TINYINFER_DECODE_SPIN).
 * The environment is read once, at the first call that needs an option; set
 * changes a value for every later call (atomically; a call already inside
 * the library may see either value).  TI_ERR_INVALID_ARG for an unknown name
 * or a value outside the option's range. No reference counterpart (kernel
 * choice and tuning for tests and benchmarks).
 */
int tinyinfer_mxfp4_set_option(const char* name, int value);
int tinyinfer_mxfp4_get_option(const char* name, int* value);

/*
 * Split-K workspaces (fp32 partial sums of the tile and GEMM kernels): the
 * bytes held over all devices and streams, and the limit of one buffer
 * (TINYINFER_WORKSPACE_MB; a call that would need more runs a kernel
 * without one, or with fewer K ranges). No reference counterpart.
 */
int tinyinfer_mxfp4_workspace_info(size_t* bytes_held, size_t* limit_bytes);

/*
 * Synchronizes every device that holds a workspace and frees them all.  No
 * graph captured before the call may be replayed after it (captured kernels
 * hold the workspace's address). No reference counterpart.
 */
int tinyinfer_mxfp4_release_workspaces(void);

/* Human-readable text for a TI_* status code (static storage). */
const char* tinyinfer_mxfp4_status_string(int status);

/* ABI version of this library (increments on any signature change). */
int tinyinfer_mxfp4_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* TINYINFER_MXFP4_H_ */
