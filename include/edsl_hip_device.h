/*
 * edsl_hip_device.h -- device-resident, asynchronous entry points.
 *
 * No counterpart in the reference: its GPU path copies every operand in and
 * out and synchronises after each of its three launches
 * (reference cpp/src/MLIRCompiler.cpp:367-454, cpp/src/MLIRExecutor.cpp:211-214).
 * These entry points are for callers that keep tensors resident in HBM and own
 * their streams: benchmark harnesses timing the kernel with stream events, and
 * chains of dense layers whose intermediates never leave the device
 * (reference tests/linalg/test_binary_op_execution.py:223-268 builds such chains).
 *
 * All pointers are device pointers; ld* are row strides in elements (inner
 * stride 1). Work is enqueued on `stream` (a hipStream_t; NULL = null stream)
 * and the call returns without waiting. Returns 0 on success, otherwise an
 * error code with the message in edsl_hip_last_error(). Library-owned
 * workspaces (small-M split-K partials, int8 operand copies) are shared by all
 * calls on a device. While one stream uses them nothing is added; the first
 * call from a second stream waits for the device once (hipDeviceSynchronize,
 * so it must not be issued during stream capture), and from then on calls
 * that use a workspace record an event that the next such call from another
 * stream waits for: those calls run one after another on the device.
 *
 * The launches may be captured into a HIP graph (stream capture) once the
 * same shapes have run eagerly, which sizes the workspaces: nothing is then
 * allocated or synchronised during capture, and workspaces that later grow
 * keep their old buffers, so a replay still finds the ones it was captured
 * with. Replays are ordered only by the stream the graph is launched on.
 */
#ifndef EDSL_HIP_DEVICE_H
#define EDSL_HIP_DEVICE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Epilogue codes: bit 0 = add bias[N]; bits 1-2 = activation: ReLU as
 * arith.maximumf (NaN propagates), leaky ReLU (f32 only), or ReLU as the
 * tensor_map body If(v > 0, v, 0) (cmpf ogt: NaN and -0 give +0; on i32 the
 * same as EDSL_EPI_RELU). */
#define EDSL_EPI_NONE 0
#define EDSL_EPI_BIAS 1
#define EDSL_EPI_RELU 2
#define EDSL_EPI_BIAS_RELU 3
#define EDSL_EPI_LEAKY 4
#define EDSL_EPI_BIAS_LEAKY 5
#define EDSL_EPI_IF_RELU 6
#define EDSL_EPI_BIAS_IF_RELU 7

/* Y[M,N] = epilogue(X[M,K] @ W[K,N] (+ bias)), f32. */
int edsl_hip_dense_f32_launch(const float *X, int64_t ldx, const float *W, int64_t ldw,
                              const float *bias, float *Y, int64_t ldy, int64_t M,
                              int64_t N, int64_t K, int epilogue, float alpha, void *stream);

/* Allocation-free variant of edsl_hip_dense_f32_launch: same arguments,
 * kernels and results (bit for bit, for the same plan). No counterpart in the
 * reference: it is for callers that cannot allocate device memory -- code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc. It calls no hipMalloc/hipFree and creates no events: the
 * small-M plan's scratch (its split-K partials) lives in a static device array of EDSL_NOALLOC_SCRATCH_BYTES
 * per GPU, held until the process ends. A plan that needs more scratch than
 * that is rejected (error code -5, the message gives both sizes); the tiled
 * plans need none. Every call on a GPU shares that GPU's array: calls that
 * overlap on one GPU (two streams or threads without ordering between them)
 * race. */
#define EDSL_NOALLOC_SCRATCH_BYTES (16u << 20)
int edsl_hip_dense_f32_launch_noalloc(const float *X, int64_t ldx, const float *W, int64_t ldw,
                                      const float *bias, float *Y, int64_t ldy, int64_t M,
                                      int64_t N, int64_t K, int epilogue, float alpha,
                                      void *stream);

/* The reference's unfused GPU sequence for the same layer, on this
 * library's kernels: a fill of Y with zeros (linalg.fill), the GEMM with no
 * epilogue, then a separate elementwise bias + activation kernel over Y --
 * the three launches the reference's GPU pipeline runs per dense layer
 * (reference cpp/src/MLIRLowering.cpp:495-518,
 * tests/gpu/test_gpu_execution.py:149-154). For measuring what fusion saves;
 * results equal edsl_hip_dense_f32_launch's bit for bit. */
int edsl_hip_dense_f32_launch_unfused(const float *X, int64_t ldx, const float *W, int64_t ldw,
                                      const float *bias, float *Y, int64_t ldy, int64_t M,
                                      int64_t N, int64_t K, int epilogue, float alpha,
                                      void *stream);

/* Y[M,N] = epilogue(X[M,K] @ W[K,N] (+ bias)), i32 wrapping arithmetic.
 * Leaky epilogues are rejected (float-only in the reference). */
int edsl_hip_dense_i32_launch(const int32_t *X, int64_t ldx, const int32_t *W, int64_t ldw,
                              const int32_t *bias, int32_t *Y, int64_t ldy, int64_t M,
                              int64_t N, int64_t K, int epilogue, void *stream);

/* Description of the kernels the calling thread's last call launched, e.g.
 * "gemm_f32 cfg=f32_256x256x16_w4x4 grid=256" (a "_edge" suffix: partial
 * edge tiles), "gemv_f32 mb=1 ksplit=4 cols=128 grid=256 +reduce" (with
 * "+xunaligned": X rows read with 4-byte loads; "+ktail": the reduce kernel adds
 * the last K % 16 rows) or "narrow_i8+gemm_i8 variant=3 waves=ksplit depth=2
 * grid=256"; returns its length. */
int edsl_hip_last_plan(char *buf, size_t len);

/* Tuning overrides: force an f32 tile configuration (index into the table
 * reported by edsl_hip_f32_config_name; -1 = automatic), the small-M
 * split-K factor (0 = automatic, at most 16) and the int8 GEMM variant.
 * Calls that cannot use the forced choice fall back to the automatic one. */
void edsl_hip_set_f32_config(int cfg);
void edsl_hip_set_gemv_ksplit(int ksplit);
/* Small-M column block: columns per workgroup, one of 32, 64, 128, 256;
 * 0 = automatic. */
void edsl_hip_set_gemv_cols(int cols);
/* Small-M kernel choice for M <= 64: 0 = automatic (the kernel or the tiles,
 * by shape), 1 = the small-M kernel whenever it can plan the layer. */
void edsl_hip_set_small_m(int mode);
/* int8 GEMM variant = wave layout and operand prefetch depth in 32-k steps:
 * 0..2 give each of 4 waves a 64x64 quadrant of the 128x128 tile, depth
 * 0: 4, 1: 2, 2: 8 when K % 256 == 0, else 4; 3 gives each wave the whole
 * tile on every fourth 32-k step (partials summed in LDS), depth 2 when
 * K/128 is even, else 1.
 * index < edsl_hip_i8_variant_count(); -1 = automatic. */
void edsl_hip_set_i8_variant(int variant);
int edsl_hip_i8_variant_count(void);
int edsl_hip_f32_config_count(void);
int edsl_hip_f32_config_name(int cfg, char *buf, size_t len);

#ifdef __cplusplus
}
#endif

#endif /* EDSL_HIP_DEVICE_H */
