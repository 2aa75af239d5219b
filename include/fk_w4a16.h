/*
 * fk_w4a16.h - C ABI of the MI355X (gfx950) W4A16 decode-linear library, libfk_w4a16.so.
 *
 * Drop-in boundary for the reference's ARC W4A16 path. Each fk_* function below replaces the
 * reference C++ op of the same name (minus the fk_ prefix) declared in
 * csrc/ops/decode_quant_linear/arc_w4a16.h:8-52 and implemented in
 * csrc/kernels/decode_quant_linear/arc_w4a16.cu:649-828; the pybind11 module
 * csrc/bindings/python_module.cpp:119-240 binds them under the same names. Argument order and
 * meaning are unchanged. Differences at the ABI level only:
 *   - device buffers are plain pointers (the reference passes std::uintptr_t), the HIP stream is a
 *     hipStream_t passed as void* (0/NULL = the null stream);
 *   - C++ exceptions become return codes: FK_OK, FK_ERR_INVALID_ARGUMENT (reference:
 *     std::invalid_argument, raised before any device work) or FK_ERR_RUNTIME (reference:
 *     std::runtime_error from CUDA / cuBLASLt); fk_last_error() returns the message of the last
 *     failure on the calling thread.
 *
 * Layouts (all row-major, little-endian):
 *   q_u8     uint8 [N, K/2]   byte b of row n holds code k=2b in bits 0-3, k=2b+1 in bits 4-7
 *   alpha    fp16  [N, K/G]   per-group scale;  beta fp16 [N, K/G] per-group offset
 *            weight value W[n,k] = alpha[n,k/G] * q[n,k] + beta[n,k/G]
 *   packets  uint8 [(N/128)*(K/G), 128*G/2 + 512]; packet (tile t, group g) is row t*(K/G)+g:
 *            code word w (codes 8w..8w+7 of the group) of column c at byte (w*128 + c)*4, then
 *            alpha[128], then beta[128] (fp16)
 *   activations [M, K] fp16 (bf16 where stated), output [M, N] in the activation dtype
 * All launches are asynchronous on the given stream; nothing synchronises the host.
 */
#ifndef FK_W4A16_H_
#define FK_W4A16_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FK_OK 0
#define FK_ERR_INVALID_ARGUMENT 1
#define FK_ERR_RUNTIME 2

#define FK_ACT_F16 0
#define FK_ACT_BF16 1

/* Message of the last failed call on this thread ("" if none). Valid until the next fk_* call. */
const char* fk_last_error(void);

/* Library version and target, e.g. "0.1.0 gfx950". */
const char* fk_build_info(void);

/* Reference: pack_arc_w4a16_packets, arc_w4a16.h:8-10 / arc_w4a16.cu:649-669. */
int fk_pack_arc_w4a16_packets(const void* q, const void* alpha, const void* beta, void* packets,
                              int n, int k, int group_size, int packet_stride_bytes, void* stream);

/* Reference: compute_arc_w4a16_group_sums, arc_w4a16.h:12-13 / arc_w4a16.cu:671-685.
 * sums[b, g] = sum over the group of x[b, k], fp32. */
int fk_compute_arc_w4a16_group_sums(const void* activations, void* sums, int batch, int k,
                                    int group_size, void* stream);

/* Reference: arc_w4a16_forward, arc_w4a16.h:15-17 / arc_w4a16.cu:687-707.
 * group_sums is accepted for signature compatibility and not read (may be NULL): the kernel forms
 * the activation sums it needs itself, in the same launch. Uses a library-owned split-K workspace
 * per (device, stream): calls on different streams never share one, and the first call of a
 * larger shape on a stream allocates (so it must not be the first call under graph capture). */
int fk_arc_w4a16_forward(const void* activations, const void* packets, const void* group_sums,
                         void* output, int batch, int n, int k, int group_size,
                         int packet_stride_bytes, void* stream);

/* Reference: arc_w4a16_forward_split_k, arc_w4a16.h:19-22 / arc_w4a16.cu:709-737.
 * Writes fp32 partials[S, batch, n]; slice z covers groups [z*ceil(NG/S), (z+1)*ceil(NG/S)).
 * group_sums is not read (may be NULL). */
int fk_arc_w4a16_forward_split_k(const void* activations, const void* packets,
                                 const void* group_sums, void* partials, int batch, int n, int k,
                                 int group_size, int packet_stride_bytes, int split_k_slices,
                                 void* stream);

/* Reference: reduce_arc_w4a16_split_k_partials, arc_w4a16.h:24-26 / arc_w4a16.cu:739-751. */
int fk_reduce_arc_w4a16_split_k_partials(const void* partials, void* output, int batch, int n,
                                         int split_k_slices, void* stream);

/* Reference: dequant_w4a16_to_fp16, arc_w4a16.h:28-30 / arc_w4a16.cu:753-770. */
int fk_dequant_w4a16_to_fp16(const void* q, const void* alpha, const void* beta, void* output,
                             int n, int k, int group_size, void* stream);

/* Reference: dequant_arc_w4a16_packets_to_fp16, arc_w4a16.h:32-34 / arc_w4a16.cu:772-789. */
int fk_dequant_arc_w4a16_packets_to_fp16(const void* packets, void* output, int n, int k,
                                         int group_size, int packet_stride_bytes, void* stream);

/* Vendor baseline. Reference: cublaslt_fp16_with_weight / _after_packet_dequant / _after_dequant,
 * arc_w4a16.h:36-52 / arc_w4a16.cu:791-828; served by hipBLASLt (fp16 in, fp32 compute). */
int fk_hipblaslt_fp16_with_weight(const void* activations, const void* weight, void* output,
                                  void* workspace, size_t workspace_bytes, int batch, int n, int k,
                                  void* stream);
int fk_hipblaslt_fp16_after_packet_dequant(const void* activations, const void* packets,
                                           void* output, void* weight, void* workspace,
                                           size_t workspace_bytes, int batch, int n, int k,
                                           int group_size, int packet_stride_bytes, void* stream);
int fk_hipblaslt_fp16_after_dequant(const void* activations, const void* q, const void* alpha,
                                    const void* beta, void* output, void* weight, void* workspace,
                                    size_t workspace_bytes, int batch, int n, int k,
                                    int group_size, void* stream);

/* ---- additions with no reference counterpart (BASELINE extensions of the same path) ------ */

typedef struct fk_arc_w4a16_plan {
  int m_tile;                /* activation rows per 128-column tile */
  int workgroups;            /* grid size */
  int groups_per_workgroup;  /* run of (tile, group) units each workgroup streams */
  int max_tile_contributors; /* workgroups that can share one slice (1 = none shared); on the
                                matrix-core stream schedule (m_tile 16, no pieces) the K parts */
  size_t workspace_bytes;    /* workspace fk_arc_w4a16_forward_ex needs */
  int slice_cols;            /* columns per workgroup unit: 128, 64, 32 or 16 */
  int schedule;              /* FK_SCHEDULE_*: how the workgroups walk their units */
} fk_arc_w4a16_plan;

/* Plan schedules. FK_SCHEDULE_RUNS: each workgroup streams runs of one slice (or tile) at a time.
 * FK_SCHEDULE_PAIRS: one-row native plans, each workgroup streams two adjacent whole 32-column
 * slices at once (slice_cols 64). FK_SCHEDULE_STREAM: one-row native plans, the whole activation
 * row staged in LDS (K <= 32768), one workgroup per CU or per slice: each workgroup streams its
 * whole slices as one contiguous range across slice boundaries, plus, when the slices do not
 * divide over the CUs, one piece of a left-over slice (groups_per_workgroup is then not a
 * multiple of K/G; the pieces are finished through the workspace). With at most half as many
 * 32-column slices as CUs (G = 128) a workgroup streams half a slice (slice_cols 16). The same
 * schedule serves one row over reference packets (whole 128-column tiles, 32-column packet
 * quarters or 16-column eighths) and 2-16 rows on the matrix cores (m_tile 16, native slabs or
 * packet quarters; K in max_tile_contributors parts when rows are too long to stage whole, the
 * parts' fp32 sums then added by a second launch). */
#define FK_SCHEDULE_RUNS 0
#define FK_SCHEDULE_PAIRS 1
#define FK_SCHEDULE_STREAM 2

/* Launch plan for a shape. split_k_slices = 0 selects the built-in policy (one resident round of
 * equal runs); S > 0 gives every workgroup ceil(K/G/S) groups. cu_count = 0 queries the current
 * device; a positive cu_count plans without touching the GPU. */
int fk_arc_w4a16_plan_for(int batch, int n, int k, int group_size, int activation_dtype,
                          int split_k_slices, int cu_count, fk_arc_w4a16_plan* plan);

/* Packet GEMV in one launch with fp16 or bf16 activations (FK_ACT_*), output in the same dtype,
 * and a caller-owned workspace: at least plan.workspace_bytes, 256-byte aligned, zero-filled
 * before its first use (every call leaves it zero-filled). Calls sharing a workspace must be
 * stream-ordered. Capturable into a HIP graph (no allocation, no memset). */
int fk_arc_w4a16_forward_ex(const void* activations, const void* packets, void* output,
                            void* workspace, size_t workspace_bytes, int batch, int n, int k,
                            int group_size, int packet_stride_bytes, int activation_dtype,
                            int split_k_slices, void* stream);

/* Native packet formats for gfx950. The reference packet interleaves the 128 columns of a tile
 * word row by word row, so a workgroup that owns fewer than 128 columns reads 128 bytes out of
 * every 512; and it stores an fp16 beta that int4 quantisation always fixes as
 * half_rn(-alpha * zp). The native formats store one slab per (128-column tile, 32-column slice,
 * group), in [tile][slice][group] order, so the groups of a slice are one contiguous byte range:
 *   code words  G/8 words (8 codes along K each) per column, in "quarter" order: column
 *               16i + n has four quarters of G/32 words; lane 16t + n of a 64-lane wave owns
 *               quarter t of columns n and n + 16. G = 128: quarter t of column 16i + n is the
 *               16 bytes at i*1024 + (16t + n)*16; G = 64: both of a lane's units share the
 *               16 bytes at (16t + n)*16 (column n first).
 *   records     16, one per column pair (n, n + 16): the two fp16 alphas (4 bytes), and for
 *               FK_PACKET_NATIVE_ASYM the two negated zero points as fp16 (-zp[n], -zp[n + 16];
 *               zp = 0 is stored as -0) (8 bytes per record).
 * FK_PACKET_NATIVE_SYM slabs are 16*G + 64 bytes (zp = 8 for every group), FK_PACKET_NATIVE_ASYM
 * slabs 16*G + 128 bytes; a buffer holds (N/32) * (K/G) slabs. (FK_PACKET_ARC is the reference
 * layout above, 64*G + 512 bytes per packet.) The forward over native slabs returns, bit for
 * bit, what it returns over the reference packets they were converted from. */
#define FK_PACKET_ARC 0
#define FK_PACKET_NATIVE_SYM 1
#define FK_PACKET_NATIVE_ASYM 2

/* Bytes per packet (FK_PACKET_ARC) or slab (native formats) for group_size 64 or 128; -1 on
 * invalid arguments. */
int fk_packet_stride_bytes(int group_size, int packet_format);

/* Native packets from q_u8 [N, K/2], alpha fp16 [N, K/G] and, for FK_PACKET_NATIVE_ASYM,
 * zero_points uint8 [N, K/G] holding 0..15 (zero_points may be NULL for the symmetric format). */
int fk_pack_native_w4a16_packets(const void* q, const void* alpha, const void* zero_points,
                                 void* packets, int n, int k, int group_size, int packet_format,
                                 void* stream);

/* Reference packets -> native packets. FK_ERR_INVALID_ARGUMENT when some beta is not
 * half_rn(-alpha * zp) for an integer zp in 0..15 (zp = 8 for the symmetric format). Synchronises
 * the stream to read the check's flag back, so it is a load-time call, not a graph node. */
int fk_convert_arc_to_native_packets(const void* arc_packets, void* native_packets, int n, int k,
                                     int group_size, int packet_format, void* stream);

/* Native packets -> reference packets, bit for bit the inverse of the conversion above. */
int fk_convert_native_to_arc_packets(const void* native_packets, void* arc_packets, int n, int k,
                                     int group_size, int packet_format, void* stream);

/* Launch plan of fk_arc_w4a16_forward_native for a packet format (arguments as
 * fk_arc_w4a16_plan_for). For the native formats below 16 activation rows slice_cols is 32, or
 * for one activation row 64 when a workgroup streams two adjacent 32-column slabs at once and 16
 * when it streams half of each slab. */
int fk_w4a16_plan_for_format(int batch, int n, int k, int group_size, int activation_dtype,
                             int split_k_slices, int cu_count, int packet_format,
                             fk_arc_w4a16_plan* plan);

/* fk_arc_w4a16_forward_ex over packets of any FK_PACKET_* format: same workspace contract
 * (workspace_bytes from fk_w4a16_plan_for_format), graph-capture behaviour and results. */
int fk_arc_w4a16_forward_native(const void* activations, const void* packets, void* output,
                                void* workspace, size_t workspace_bytes, int batch, int n, int k,
                                int group_size, int packet_format, int activation_dtype,
                                int split_k_slices, void* stream);

/* fk_arc_w4a16_forward_native with the automatic plan, for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. It takes no workspace and calls no hipMalloc / hipFree: the stream-K fix-up scratch
 * is a file-scope device array of FK_NOALLOC_SCRATCH_BYTES that every GPU the library runs on
 * holds until the process ends, set up on the first call on a device (address lookup and one
 * clearing kernel on that call's stream). Launches whose plan needs more scratch than that fail
 * with FK_ERR_INVALID_ARGUMENT before any device work. Every call on one GPU shares its array:
 * calls that overlap on one GPU (different streams, graphs replayed concurrently) race; calls
 * ordered on one stream do not. As a guard, a call whose plan uses the scratch fails with
 * FK_ERR_RUNTIME when the previous such call on that GPU came from another stream that still has
 * work queued (not checked while the calling stream is being captured). Results are those of
 * fk_arc_w4a16_forward_native. */
#define FK_NOALLOC_SCRATCH_BYTES (8388608 + 65536)
int fk_w4a16_forward_noalloc(const void* activations, const void* packets, void* output, int batch,
                             int n, int k, int group_size, int packet_format,
                             int activation_dtype, void* stream);

/* Kernel choice for fk_w4a16_plan_for_kernel / fk_w4a16_forward_kernel. No counterpart in the
 * reference; they succeed the reference's per-kernel suite ids (decode/w4a16_linear_scalar and the
 * tensor-core ids), so that the suites can time one kernel against another:
 *   FK_KERNEL_AUTO  the dispatch of fk_arc_w4a16_forward_native (dot2 loop below 8 activation
 *                   rows, the matrix-core kernel from 8);
 *   FK_KERNEL_DOT2  the dot2 loop for every batch (m-tiles of at most 8 rows);
 *   FK_KERNEL_MFMA  the matrix-core kernel for every batch (16-row m-tiles, 128-column tiles). */
#define FK_KERNEL_AUTO 0
#define FK_KERNEL_DOT2 1
#define FK_KERNEL_MFMA 2

/* fk_w4a16_plan_for_format / fk_arc_w4a16_forward_native with a kernel choice; same workspace
 * contract (workspace_bytes from fk_w4a16_plan_for_kernel with the same choice). */
int fk_w4a16_plan_for_kernel(int batch, int n, int k, int group_size, int activation_dtype,
                             int split_k_slices, int cu_count, int packet_format, int kernel,
                             fk_arc_w4a16_plan* plan);
int fk_w4a16_forward_kernel(const void* activations, const void* packets, void* output,
                            void* workspace, size_t workspace_bytes, int batch, int n, int k,
                            int group_size, int packet_format, int activation_dtype,
                            int split_k_slices, int kernel, void* stream);

/* Fused decode-step neighbours over native slabs (FK_PACKET_NATIVE_SYM / _ASYM); no counterpart
 * in the reference, whose decode step runs these as separate launches.
 *
 * fk_w4a16_forward_rmsnorm: y = x_n . W^T with x_n = round(gamma * round(x * rsqrt(mean(x^2) +
 * eps))) in the activation dtype (the Llama input RMSNorm of the qkv / gate_up projections,
 * rounded as an unfused norm kernel writing x_n would round it); norm_weight = gamma [K] in the
 * activation dtype. Workspace: at least plan.workspace_bytes from fk_w4a16_plan_rmsnorm, with the
 * contract of fk_arc_w4a16_forward_ex. */
int fk_w4a16_plan_rmsnorm(int batch, int n, int k, int group_size, int activation_dtype,
                          int split_k_slices, int cu_count, int packet_format,
                          fk_arc_w4a16_plan* plan);
int fk_w4a16_forward_rmsnorm(const void* activations, const void* norm_weight, float eps,
                             const void* packets, void* output, void* workspace,
                             size_t workspace_bytes, int batch, int n, int k, int group_size,
                             int packet_format, int activation_dtype, int split_k_slices,
                             void* stream);

/* fk_w4a16_forward_silu_mul: the gate_up projection with its activation. The slabs hold
 * [W_gate; W_up] stacked along n (n % 256 == 0); output [batch, n/2] =
 * round(round(silu(round(x . W_gate^T))) * round(x . W_up^T)) in the activation dtype, one
 * launch, no workspace. A non-NULL norm_weight applies the RMSNorm prologue of
 * fk_w4a16_forward_rmsnorm to x first (a Llama block's norm, gate_up and SiLU in one launch). */
int fk_w4a16_forward_silu_mul(const void* activations, const void* packets, void* output,
                              int batch, int n, int k, int group_size, int packet_format,
                              int activation_dtype, const void* norm_weight, float eps,
                              void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FK_W4A16_H_ */
