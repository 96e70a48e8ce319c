/*
 * convnd_hip.h — C ABI of the MI355X (gfx950) N-d dense convolution library.
 *
 * Plain pointers, sizes and a stream handle: no torch types cross this boundary.
 * Every tensor argument is a dense, row-major (C-contiguous) device buffer:
 *   input        [batch, channels, input[0], ..., input[rank-1]]
 *   weight       [output_channels, channels / groups, kernel[0], ..., kernel[rank-1]]
 *   bias         [output_channels]                      (nullable)
 *   output       [batch, output_channels, out[0], ..., out[rank-1]]
 * with out[a] = (input[a] + 2*padding[a] - dilation[a]*(kernel[a]-1) - 1) / stride[a] + 1.
 * All tensors share one element type (convnd_hip_dtype). Work is enqueued on `stream`
 * (a hipStream_t; NULL is the default stream) and nothing synchronises the host.
 * Results are deterministic: no floating-point atomics are used anywhere.
 *
 * Each entry point names the reference interface it replaces (lyehe/torch-convnd,
 * paths relative to the reference repository).
 */
#ifndef CONVND_HIP_H
#define CONVND_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* PyTorch tensors have at most 64 dimensions: batch, channels and 62 spatial axes
 * (src/torch_convnd/csrc/convnd.h:10-11). */
#define CONVND_HIP_MAX_RANK 62

typedef enum convnd_hip_dtype {
  CONVND_HIP_FLOAT32 = 0,
  CONVND_HIP_FLOAT64 = 1,
  CONVND_HIP_FLOAT16 = 2,
  CONVND_HIP_BFLOAT16 = 3
} convnd_hip_dtype;

/* Activation fused into the forward epilogue (convnd_hip_forward_act). GELU is the exact
 * (erf) form, GELU_TANH its tanh approximation, as torch.nn.functional.gelu with
 * approximate="none" / "tanh". */
typedef enum convnd_hip_activation {
  CONVND_HIP_ACT_NONE = 0,
  CONVND_HIP_ACT_RELU = 1,
  CONVND_HIP_ACT_GELU = 2,
  CONVND_HIP_ACT_GELU_TANH = 3
} convnd_hip_activation;

/* Memory layout of the activation tensors of a call (input, output, grad_output and
 * grad_input; weights are always [output_channels, channels / groups, kernel...]):
 *   CHANNELS_FIRST  [batch, channels, spatial...]  (the reference's only layout)
 *   CHANNELS_LAST   [batch, spatial..., channels]  (channels innermost, as PyTorch's
 *                   channels_last / channels_last_3d memory formats and their N-d analogue)
 *   CHANNELS_LAST_INPUT  input channels-last; output, grad_output and grad_input
 *                   channels-first. This is what the reference operators give a channels-last
 *                   input: they read it through a contiguous copy and return contiguous
 *                   results (src/torch_convnd/csrc/convnd.cpp:317-320,377-386). Here the
 *                   forward GEMM reads the channels-last input itself where it can. */
typedef enum convnd_hip_layout {
  CONVND_HIP_CHANNELS_FIRST = 0,
  CONVND_HIP_CHANNELS_LAST = 1,
  CONVND_HIP_CHANNELS_LAST_INPUT = 2
} convnd_hip_layout;

typedef enum convnd_hip_status {
  CONVND_HIP_SUCCESS = 0,
  CONVND_HIP_INVALID_ARGUMENT = 1, /* geometry/shape/dtype rejected; see convnd_hip_last_error */
  CONVND_HIP_WORKSPACE_TOO_SMALL = 2,
  CONVND_HIP_LAUNCH_FAILED = 3,    /* a HIP call failed; message holds hipGetErrorString */
  CONVND_HIP_UNSUPPORTED = 4
} convnd_hip_status;

/* Convolution problem description. Replaces the `Geometry` struct and the tensor
 * metadata that `make_geometry` reads (src/torch_convnd/csrc/convnd.h:13-27,
 * src/torch_convnd/csrc/convnd.cpp:33-87). Only the first `rank` entries of each array
 * are read. */
typedef struct convnd_hip_problem {
  int64_t rank;            /* spatial rank, 1..62 */
  int64_t batch;           /* N >= 0 */
  int64_t channels;        /* input channels C */
  int64_t output_channels; /* Co */
  int64_t groups;          /* G; C and Co divisible by G */
  int64_t input[CONVND_HIP_MAX_RANK];
  int64_t kernel[CONVND_HIP_MAX_RANK];
  int64_t stride[CONVND_HIP_MAX_RANK];
  int64_t padding[CONVND_HIP_MAX_RANK]; /* symmetric zero padding */
  int64_t dilation[CONVND_HIP_MAX_RANK];
} convnd_hip_problem;

/* Human-readable message of the last failure on the calling thread ("" if none).
 * Messages reuse the reference's wording, e.g. "groups must be positive",
 * "kernel exceeds padded input", "workspace_bytes is too small for one output position". */
const char* convnd_hip_last_error(void);

/* Validates the geometry and the workspace_bytes contract and writes the output
 * spatial sizes (`rank` entries) to `output_sizes` (nullable).
 * Replaces make_geometry + tile_size (src/torch_convnd/csrc/convnd.cpp:33-100):
 * workspace_bytes must be >= max(element_size, 4) * channels * prod(kernel), as in the
 * reference, although the implicit GEMM below needs no patch buffer.
 * Touches no device; safe to call on a machine without a GPU. */
int convnd_hip_validate(const convnd_hip_problem* problem, int64_t element_size,
                        int64_t workspace_bytes, int64_t* output_sizes);

/* Device scratch bytes convnd_hip_forward needs for this problem (0 is possible). */
size_t convnd_hip_forward_workspace_size(const convnd_hip_problem* problem,
                                         convnd_hip_dtype dtype);

/* output = conv(input, weight) + bias. Replaces the CUDA forward driver `conv_nd`
 * (src/torch_convnd/csrc/convnd.cpp:305-343) together with its unfold kernels
 * (src/torch_convnd/csrc/convnd_cuda.cu:91-145,173-191) and GEMM call (convnd.cpp:334):
 * an implicit GEMM on MFMA for bf16/fp16/fp32 when the channel layout allows, a direct
 * kernel otherwise. `workspace` must hold convnd_hip_forward_workspace_size bytes. */
int convnd_hip_forward(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                       const void* input, const void* weight, const void* bias, void* output,
                       void* workspace, size_t workspace_size, void* stream);

/* output = act(conv(input, weight) + bias), the activation applied in the GEMM epilogue
 * (in fp32, fp64 for fp64) before the single rounding to the element type; with
 * CONVND_HIP_ACT_NONE it is convnd_hip_forward. Kernels without a fused epilogue (the
 * direct fallback) apply it in one more elementwise pass. Same workspace as
 * convnd_hip_forward. No reference counterpart: the reference runs the activation as a
 * separate PyTorch launch after its bias epilogue (src/torch_convnd/csrc/convnd.cpp:337-341;
 * README.md:129-138 shows the Conv4d -> GELU -> Conv4d stack). */
int convnd_hip_forward_act(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                           const void* input, const void* weight, const void* bias,
                           void* output, int activation, void* workspace,
                           size_t workspace_size, void* stream);

/* Device scratch bytes convnd_hip_backward needs for the requested gradients. */
size_t convnd_hip_backward_workspace_size(const convnd_hip_problem* problem,
                                          convnd_hip_dtype dtype, int need_grad_input,
                                          int need_grad_weight, int need_grad_bias);

/* Gradients of conv(input, weight) + bias for a cotangent grad_output. A NULL
 * grad_input / grad_weight / grad_bias skips that gradient (the reference's
 * output_mask). Every requested gradient buffer is fully overwritten (no accumulation).
 * Low-precision gradients accumulate in fp32 and are rounded once to the element type.
 * Replaces `conv_nd_backward` and `mixed_backward_cuda`
 * (src/torch_convnd/csrc/convnd.cpp:345-415, src/torch_convnd/csrc/convnd_mixed.cpp:11-60)
 * with their fold kernels (src/torch_convnd/csrc/convnd_cuda.cu:147-169,193-213). */
int convnd_hip_backward(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                        const void* grad_output, const void* input, const void* weight,
                        void* grad_input, void* grad_weight, void* grad_bias, void* workspace,
                        size_t workspace_size, void* stream);

/* Device scratch bytes of convnd_hip_forward_layout / convnd_hip_backward_layout for a
 * layout (CHANNELS_FIRST: the same as convnd_hip_forward_workspace_size /
 * convnd_hip_backward_workspace_size). */
size_t convnd_hip_forward_workspace_size_layout(const convnd_hip_problem* problem,
                                                convnd_hip_dtype dtype, int layout);
size_t convnd_hip_backward_workspace_size_layout(const convnd_hip_problem* problem,
                                                 convnd_hip_dtype dtype, int layout,
                                                 int need_grad_input, int need_grad_weight,
                                                 int need_grad_bias);

/* convnd_hip_forward_act / convnd_hip_backward with the activation tensors in `layout`
 * (convnd_hip_layout). With CHANNELS_LAST the implicit GEMM with direct staging (16-bit data)
 * reads [batch, spatial..., channels] and writes [batch, out..., output_channels] itself, so
 * such a forward makes no layout copy; other plans, and the weight gradient (whose kernels
 * read channels-first operands), run on channels-first copies in the workspace. With
 * CHANNELS_LAST_INPUT the same GEMM reads the channels-last input and writes a channels-first
 * output; the backward is the channels-first one with the weight gradient reading a
 * channels-first copy of the input. Results are the same numbers as the channels-first call.
 * CHANNELS_LAST_INPUT is the layout of the reference operators' contract for a channels-last
 * input (they copy every operand to channels-first and return channels-first results,
 * src/torch_convnd/csrc/convnd.cpp:317-320,377-386); CHANNELS_LAST has no reference
 * counterpart. */
int convnd_hip_forward_layout(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                              int layout, int activation, const void* input, const void* weight,
                              const void* bias, void* output, void* workspace,
                              size_t workspace_size, void* stream);
int convnd_hip_backward_layout(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                               int layout, const void* grad_output, const void* input,
                               const void* weight, void* grad_input, void* grad_weight,
                               void* grad_bias, void* workspace, size_t workspace_size,
                               void* stream);

/* Partial convolution's counts: window sums of a validity map under the convolution's
 * geometry (a depthwise all-ones convolution with symmetric zero padding). Reads
 * problem->rank (1..8), batch, channels (the map's channels), groups (count channels,
 * dividing channels), input, kernel, stride, padding and dilation; output_channels is
 * ignored. mask [batch, channels, input...] of `mask_dtype`; counts [batch, groups, out...]
 * float32 (float64 when mask_dtype is CONVND_HIP_FLOAT64); count channel q sums map
 * channels [q*channels/groups, (q+1)*channels/groups) over each window's in-bounds taps.
 * Replaces _count / _counting_kernel and the per-group channel sum of multi-channel masks
 * (src/torch_convnd/functional.py:395-441,536-545), which run a convolution through the
 * native operator. */
int convnd_hip_partial_count(const convnd_hip_problem* problem, convnd_hip_dtype mask_dtype,
                             const void* mask, void* counts, void* stream);

/* Partial convolution's rescale epilogue, one pass over the raw convolution output
 * (computed without bias). For element (n, c, p), with k = counts[n', c / (channels /
 * count_channels), p] and n' = n when count_batch == batch, else 0:
 *   u = clamp(k, 0, 1), r = u * window / max(k, smallest normal)
 *   out = raw * r                   (bias NULL)
 *   out = (raw * r + bias[c]) * u   (bias given)
 * evaluated in the count type and rounded once to `dtype`.
 * raw, out [batch, channels, positions] of `dtype` (out may equal raw); bias [channels] of
 * `dtype`; counts [count_batch, count_channels, positions] float32 (float64 when dtype is
 * CONVND_HIP_FLOAT64), count_batch 1 or batch, count_channels dividing channels.
 * Replaces the elementwise rescale of partial convolution, _scale and the tail of
 * _partial_conv_nd (src/torch_convnd/functional.py:312-321,592-616), which the reference
 * runs as separate PyTorch launches. */
int convnd_hip_partial_rescale(convnd_hip_dtype dtype, const void* raw, const void* counts,
                               const void* bias, void* out, int64_t batch, int64_t channels,
                               int64_t positions, int64_t count_batch, int64_t count_channels,
                               double window, void* stream);

/* Bytes of the device scratch array convnd_hip_forward_noalloc uses, one per GPU (64 MiB). */
#define CONVND_HIP_NOALLOC_SCRATCH_BYTES (64u << 20)

/* convnd_hip_forward without a workspace and without any device allocation: the staged
 * input, the packed weights and the geometry tables live in a file-scope device array of
 * CONVND_HIP_NOALLOC_SCRATCH_BYTES per GPU, held from the library's load until the process
 * ends; the call itself makes no hipMalloc / hipFree. Problems whose scratch needs exceed it
 * fail with CONVND_HIP_WORKSPACE_TOO_SMALL and a message naming the size. Every call on one
 * GPU shares that GPU's array and leaves its contents behind (each call rewrites all it
 * reads), so calls that overlap on one GPU (other streams, other threads) race: serialise
 * them. Same results as convnd_hip_forward (the same kernels).
 * No counterpart in the reference: for callers that cannot allocate device memory -- code
 * under stream capture, serving loops that must not allocate, harnesses that forbid
 * hipMalloc. */
int convnd_hip_forward_noalloc(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                               const void* input, const void* weight, const void* bias,
                               void* output, void* stream);

/* Which kernel family convnd_hip_forward / convnd_hip_backward would use, as a short
 * string ("mfma", "direct", ...) for diagnostics and tests. `which`: 0 forward,
 * 1 input gradient, 2 weight gradient. No reference counterpart (diagnostic only). */
const char* convnd_hip_plan_name(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                                 int which);

/* Diagnostic, no counterpart in the reference: plans the forward and every gradient of a
 * problem, builds their geometry tables in host memory and checks every entry against the
 * buffer the kernels index with it (LDS halo and staging regions, tap prefetch rows, output
 * offsets, weight-packing map, weight-gradient columns and load sources). Touches no GPU.
 * Returns CONVND_HIP_SUCCESS, or CONVND_HIP_LAUNCH_FAILED with the first violation in
 * convnd_hip_last_error(). Used by the host-only sanitizer build of the tests. */
int convnd_hip_plan_check(const convnd_hip_problem* problem, convnd_hip_dtype dtype);

/* JSON description of the launch plan (kernel family, box shape, channel chunk, LDS bytes,
 * occupancy, workgroups) written to `buffer` (NUL-terminated, truncated to `length`).
 * `which`: 0 forward, 1 input gradient, 2 weight gradient. Diagnostic only, no reference
 * counterpart; touches no device. */
int convnd_hip_plan_describe(const convnd_hip_problem* problem, convnd_hip_dtype dtype,
                             int which, char* buffer, size_t length);

/* Diagnostic kernel timing, no reference counterpart. While enabled, each launch of the
 * forward implicit GEMM (kernel id 0), the input-gradient implicit GEMM (id 1) and the MFMA
 * weight-gradient kernel (id 2) is bracketed by HIP events recorded on the launch stream.
 * Process-global (any thread); not for concurrent use. */
int convnd_hip_timing_enable(int enable);

/* After the launch streams have synchronised: total milliseconds and number of timed
 * launches of kernel `kernel` since the previous read; clears that record. */
int convnd_hip_timing_read(int kernel, double* total_ms, int64_t* launches);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CONVND_HIP_H */
