/*
 * llk_abi.h -- C ABI of the MI355X (gfx950) backend for DSLCompiler's fused
 * SwiGLU / micro.mma hot path.
 *
 * Plain C: pointers, sizes and status codes; no torch or C++ types.  Every
 * entry point is declared next to the reference interface it replaces
 * (paths relative to the skg7on/DSLCompiler tree).
 *
 * Conventions
 *   - Return value: LLK_OK (0) on success, a negative llk_status on error.
 *     llk_last_error() returns a thread-local, human-readable message for the
 *     most recent failing call on the calling thread.
 *   - Launch entry points are stream-ordered and asynchronous: they enqueue
 *     on ctx->stream (NULL = the default stream) and return without waiting.
 *     All tensor data pointers passed to them are device pointers on the
 *     current HIP device.
 *   - A packed-weights handle is immutable after packing and may be shared by
 *     launches on any stream of the device it was packed for.  Freeing it
 *     while launches that use it are still queued is the caller's error.
 *   - Element types: bf16 inputs; outputs bf16 or fp32 as requested.  Tensors
 *     are 2-D with unit inner stride (stride1 == 1); stride0 is the row
 *     stride in elements and must be >= dim1.
 */
#ifndef LLK_ABI_H
#define LLK_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LLK_ABI_VERSION 4

/* Status codes.  The reference returns errors as llvm::Expected /
 * StringError (JitCache.cpp:200-224); this ABI uses negative integers. */
typedef enum llk_status {
  LLK_OK = 0,
  LLK_ERR_INVALID_ARGUMENT = -1, /* null pointer, bad enum value          */
  LLK_ERR_SHAPE = -2,            /* dimension mismatch (LLKOps.cpp:42-83)  */
  LLK_ERR_DTYPE = -3,            /* unsupported element type               */
  LLK_ERR_LAYOUT = -4,           /* stride1 != 1, stride0 < dim1, alignment */
  LLK_ERR_HIP = -5,              /* a HIP runtime call failed              */
  LLK_ERR_NO_DEVICE = -6,        /* no HIP device visible                  */
  LLK_ERR_UNSUPPORTED_ARCH = -7, /* current device is not gfx950           */
  LLK_ERR_OUT_OF_MEMORY = -8,    /* host or device allocation failed       */
  LLK_ERR_SCRATCH = -9,          /* caller scratch too small / misaligned  */
  LLK_ERR_DEVICE_MISMATCH = -10, /* handle packed for another device       */
  LLK_ERR_NOT_FOUND = -11        /* schedule DB / code object missing      */
} llk_status;

/* Element types: values of llk::DType (KernelKey.h:22). */
typedef enum llk_dtype { LLK_BF16 = 0, LLK_FP16 = 1, LLK_FP32 = 2 } llk_dtype;

/* Tensor2D (JitCache.h:30-36): same fields, same order, same meaning. */
typedef struct llk_tensor2d {
  void* data;
  int64_t dim0;
  int64_t dim1;
  int64_t stride0;
  int64_t stride1;
} llk_tensor2d;

/* KernelContext (JitCache.h:59-62) plus the HIP stream to launch on.
 * scratch/scratch_size: optional caller-owned device workspace; when
 * scratch is NULL the library uses a workspace it owns per device.  The
 * required size is given by llk_swiglu_scratch_size(). */
typedef struct llk_kernel_context {
  void* scratch;
  size_t scratch_size;
  void* stream; /* hipStream_t */
} llk_kernel_context;

/* Opaque packed-weights handle (PackedWeights, PackedWeights.h:13-43). */
typedef struct llk_packed_weights llk_packed_weights;

/* ----------------------------------------------------------------------- */
/* Library / target                                                         */
/* ----------------------------------------------------------------------- */

/* Thread-local message of the last failing call ("" if none). */
const char* llk_last_error(void);

/* LLK_ABI_VERSION of the loaded library. */
int llk_abi_version(void);

/* Device query (replaces CpuFeatures::detect / bestIsa,
 * lib/Target/X86/TargetAVX2.cpp:33-92).  Fills arch_name (NUL-terminated,
 * at most cap bytes), compute-unit count, LDS bytes per workgroup and the
 * peak engine clock in kHz of the current device.  Returns
 * LLK_ERR_UNSUPPORTED_ARCH (after filling the fields) when the device is not
 * gfx950. */
int llk_device_info(char* arch_name, int cap, int* cu_count, int* lds_bytes,
                    int* clock_khz);

/* ----------------------------------------------------------------------- */
/* Packed weights (PackedWeights.h:46-49, PackedWeights.cpp:5-37)           */
/* ----------------------------------------------------------------------- */

/* Pack flags. */
#define LLK_PACK_KEEP_HOST 1u /* also keep the reference host layout       */
#define LLK_PACK_HOST_ONLY 2u /* host layout only: no device payload, no
                                 HIP call (the reference's host-only packer);
                                 kernels reject such a handle            */

/* packWeightMatrix (PackedWeights.cpp:5-33).  `w` is a bf16 [K, N] matrix in
 * HOST memory (stride1 == 1).  Metadata follows the reference exactly:
 * N = dim1, BK = bk, K_blocks = ceil(K / BK), block_size = BK * N * 2,
 * dtype = BF16.  The device payload (on the current device) is laid out in
 * MFMA operand order: see llk_pack_device_layout.  With LLK_PACK_KEEP_HOST
 * the handle also owns the reference's host buffer [K_blocks][BK][N]
 * (zero-padded), readable through llk_packed_weights_host_data. */
int llk_pack_weights(const llk_tensor2d* w_host, int64_t bk, unsigned flags,
                     llk_packed_weights** out);

/* Same as llk_pack_weights for a bf16 [K, N] matrix already in DEVICE memory;
 * the repack runs as a kernel on `stream` and this call waits for it.
 * LLK_PACK_KEEP_HOST is not accepted here. */
int llk_pack_weights_device(const llk_tensor2d* w_dev, int64_t bk,
                            void* stream, llk_packed_weights** out);

/* repack (PackedWeights.cpp:35-37): re-pack new host contents into an
 * existing handle, keeping its BK.  The shape must be unchanged. */
int llk_repack(llk_packed_weights* pw, const llk_tensor2d* w_host);

/* Destroys the handle and frees host and device buffers.  NULL is a no-op. */
void llk_packed_weights_free(llk_packed_weights* pw);

/* Metadata getters (PackedWeights.h:13-19 fields), exact reference values. */
int64_t llk_packed_weights_k_blocks(const llk_packed_weights* pw);
int64_t llk_packed_weights_n(const llk_packed_weights* pw);
int64_t llk_packed_weights_block_size(const llk_packed_weights* pw);
int64_t llk_packed_weights_bk(const llk_packed_weights* pw);
int llk_packed_weights_dtype(const llk_packed_weights* pw);
/* The logical K (rows of the packed matrix); not a reference field. */
int64_t llk_packed_weights_k(const llk_packed_weights* pw);
/* Reference host layout, or NULL when LLK_PACK_KEEP_HOST was not given. */
const void* llk_packed_weights_host_data(const llk_packed_weights* pw);
/* Device payload pointer and size in bytes. */
const void* llk_packed_weights_device_data(const llk_packed_weights* pw);
size_t llk_packed_weights_device_bytes(const llk_packed_weights* pw);

/* Host-side implementation of the device payload layout, for inspection
 * (no HIP call): writes the device layout of bf16 [K, N] `w_host` into
 * `out`, which must hold llk_pack_device_bytes(K, N) bytes. */
size_t llk_pack_device_bytes(int64_t K, int64_t N);
int llk_pack_device_layout(const llk_tensor2d* w_host, void* out);

/* ----------------------------------------------------------------------- */
/* Kernels                                                                  */
/* ----------------------------------------------------------------------- */

/* Fused SwiGLU  Y = SiLU(X Wg) * (X Wu).
 * Replaces the JIT'd kernel `KernelFn(x, wg, wu, init, result)`
 * (JitCache.h:79-81) produced from llk.fused_swiglu (LLKOps.td:13-67) by
 * FuseDoubleContraction (FuseDoubleContraction.cpp:109-199).
 * x: bf16 [M, K] device; wg, wu: packed [K, N] handles; y: [M, N] device of
 * y_dtype LLK_BF16 (truncf RNE of the fp32 result, the reference op's result
 * type) or LLK_FP32 (the pre-truncf value).  fp32 accumulation, exact exp.
 * M == 0 is valid and launches nothing (edge_cases.cpp:84-97).  K == 0 is
 * valid (the verifier accepts an empty reduction, LLKOps.cpp:42-83) and
 * fills Y with +0: SiLU(0) * 0 of the zero-filled fp32 accumulators
 * (FuseDoubleContraction.cpp:119-135). */
int llk_swiglu_bf16(const llk_tensor2d* x, const llk_packed_weights* wg,
                    const llk_packed_weights* wu, llk_tensor2d* y, int y_dtype,
                    llk_kernel_context* ctx);

/* llk_swiglu_bf16 for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  Same arguments, checks and results as
 * llk_swiglu_bf16 (launched on `stream`, NULL = the default stream), but the
 * workspace is a fixed 64 MiB device array built into the library (one per
 * GPU, held until the process ends) instead of ctx->scratch or the library's
 * growable buffers: the call makes no hipMalloc/hipFree.  Plans that would
 * need more workspace use fewer k splits or shorter row chunks; a shape whose
 * smallest plan still needs more (a padded X with K > ~65000) returns
 * LLK_ERR_SCRATCH.  Every call on a GPU shares that array: calls that overlap
 * on one GPU (two streams, two threads) race and must be serialised by the
 * caller. */
int llk_swiglu_bf16_noalloc(const llk_tensor2d* x, const llk_packed_weights* wg,
                            const llk_packed_weights* wu, llk_tensor2d* y, int y_dtype,
                            void* stream);

/* FusedSwiGLUOp::verify (LLKOps.cpp:42-83): the same checks in the same
 * order with the same messages; a negative dimension is dynamic and skips
 * the checks it takes part in.  LLK_OK or LLK_ERR_SHAPE.  llk_swiglu_bf16
 * applies it to its arguments. */
int llk_verify_fused_swiglu(int64_t x_m, int64_t x_k, int64_t wg_k, int64_t wg_n, int64_t wu_k,
                            int64_t wu_n, int64_t init_m, int64_t init_n);
/* MatmulOp::verify (LLKOps.cpp:336-348): K of A must equal K of B. */
int llk_verify_matmul(int64_t a_k, int64_t b_k);

/* Device workspace bytes llk_swiglu_bf16 needs for an M x N problem when the
 * caller supplies ctx->scratch (0 when none is needed). */
size_t llk_swiglu_scratch_size(int64_t M, int64_t N, int64_t K);

/* The launch the dispatcher chooses for an op (llk_kernel_key operation
 * values: 0 fused SwiGLU, 3 matmul) on an M x N x K problem -- the role of
 * the reference's ShapeSpecialization + ScheduleSelection passes
 * (ShapeSpecialization.cpp:38-48, ScheduleSelection.cpp:46-67) for this
 * backend.  flags: LLK_PLAN_X_ALIGNED -- X rows are 16-byte aligned with
 * K % 8 == 0 (else the worst case, a padded copy of X, is assumed);
 * LLK_PLAN_ACCUMULATE -- the plan of llk_gemm_bf16_accumulate (matmul only),
 * which always ends with the reduce launch that adds C and needs its
 * partial planes even unsplit; LLK_PLAN_OUT_F32 -- fused SwiGLU with an fp32
 * result (the pre-truncf value) instead of the op's bf16 one.  workspace_bytes
 * is then exactly the ctx->scratch size that call needs.  Host-only, no HIP
 * call. */
#define LLK_PLAN_X_ALIGNED 1u
#define LLK_PLAN_ACCUMULATE 2u
#define LLK_PLAN_OUT_F32 4u
typedef struct llk_launch_plan {
  int kernel;                    /* 0 small-M bandwidth kernel, 1 MFMA tile kernel,
                                    2 wide SwiGLU tile kernel (bf16 result),
                                    3 decode tile kernel (M <= 64, K % 64 == 0,
                                    aligned X: LLK_PLAN_X_ALIGNED) */
  int splits;                    /* k splits across workgroups (1 = none) */
  int group_width;               /* small-M kernel: 32-column groups per workgroup */
  int pad_x;                     /* tile kernel: X copied to a padded buffer first */
  int64_t workgroups;            /* of the main kernel, per row chunk (all its launches) */
  int64_t threads_per_workgroup; /* of the main kernel */
  int64_t launches;              /* kernel launches per call */
  size_t workspace_bytes;        /* = ctx->scratch size the call needs */
  int64_t head_blocks_n;         /* tile kernel: leading 128-column blocks launched
                                    without k split before the rest takes `splits`
                                    (0 = one launch over all columns) */
  int64_t tile_columns;          /* tile kernels: output columns per workgroup (each
                                    matrix for SwiGLU); 0 for the small-M kernel */
} llk_launch_plan;
int llk_describe_launch(int operation, int64_t M, int64_t N, int64_t K, unsigned flags,
                        llk_launch_plan* out);

/* Library-owned workspaces of the current device (no reference
 * counterpart; for long-running callers that watch device memory).  When a
 * call gets no ctx->scratch, the library uses a workspace of its own per
 * stream (per thread for the per-thread default stream), grown on demand,
 * and keeps at most the tunable "max_workspaces" (default 16) per device:
 * a further stream evicts the least recently used idle one.  A buffer is
 * freed only after the last call that used it has finished on the GPU; one
 * used while its stream was capturing a HIP graph is kept until the process
 * ends.  llk_workspace_stats reports the live workspaces and their bytes;
 * llk_workspace_trim frees every idle, uncaptured one (waiting for its last
 * call). */
int llk_workspace_stats(size_t* count, size_t* bytes);
int llk_workspace_trim(void);

/* micro.mma matmul  C = A B  (MicroOps.td:196-222, MicroOps.cpp:246-291;
 * llk.matmul, LLKOps.td:210-255, accumulator f32), i.e. with a zero initial
 * accumulator; llk_gemm_bf16_accumulate below is the C += A B form.
 * a: bf16 [M, K] device; b: packed [K, N] handle; c: [M, N] device of
 * c_dtype LLK_FP32, LLK_BF16 or LLK_FP16 (the result types llk.matmul
 * allows; both 16-bit types round the fp32 sum to nearest even, fp16
 * overflows to infinity).  K == 0 (MatmulOp::verify accepts it,
 * LLKOps.cpp:336-348) fills C with +0. */
int llk_gemm_bf16(const llk_tensor2d* a, const llk_packed_weights* b,
                  llk_tensor2d* c, int c_dtype, llk_kernel_context* ctx);

/* The accumulating form  C += A B: micro.mma's  acc += lhs * rhs
 * (MicroOps.td:196-222) and llk.matmul / linalg.matmul with a non-zero
 * outs(init) (LLKOps.td:210-255).  C's existing values are read in c_dtype,
 * widened to fp32 and added to the fp32 sum of products before the result
 * is rounded to c_dtype (one rounding per call; the products are summed
 * first, then C is added).  K == 0 leaves C untouched.  Same arguments and
 * errors as llk_gemm_bf16; c is read and written in place. */
int llk_gemm_bf16_accumulate(const llk_tensor2d* a, const llk_packed_weights* b,
                             llk_tensor2d* c, int c_dtype, llk_kernel_context* ctx);

/* MLP block: Y = SwiGLU(X; Wg, Wu) in bf16, then Z = Y Wd (fp32 accumulate,
 * bf16 result).  wd is a packed [N, K_out] handle.  y is a caller-owned
 * bf16 [M, N] device buffer that receives the intermediate.  No reference
 * op (the reference has no lowering for llk.matmul: LLKToLinalg.cpp:621-646);
 * composed from the two entry points above. */
int llk_mlp_bf16(const llk_tensor2d* x, const llk_packed_weights* wg,
                 const llk_packed_weights* wu, const llk_packed_weights* wd,
                 llk_tensor2d* y, llk_tensor2d* z, llk_kernel_context* ctx);

/* ----------------------------------------------------------------------- */
/* Shape specialisation and schedules                                       */
/* ----------------------------------------------------------------------- */

/* classifyM (ScheduleLoader.cpp:19-29). */
int llk_classify_m(int64_t M);

/* TilingUtils.h:28-50. */
int64_t llk_num_tiles(int64_t dim, int64_t tile);
int64_t llk_tile_size(int64_t dim, int64_t tile, int64_t idx);
int64_t llk_num_inner_tiles(int64_t outer, int64_t inner);

/* KernelKey::hash (KernelKey.h:60-86) over the twelve fields. */
uint64_t llk_kernel_key_hash(uint8_t operation, uint8_t input_type,
                             uint8_t output_type, int64_t m_bucket, int64_t n,
                             int64_t k, uint8_t weight_layout, uint8_t isa,
                             uint8_t math_mode, uint16_t thread_count,
                             uint64_t compiler_version,
                             uint64_t schedule_version);

/* ScheduleEntry (ScheduleLoader.h:23-31). */
typedef struct llk_schedule_entry {
  int64_t BM, BN, BK, VM, VN, vector_width, num_threads, grain_size;
  char parallel_axis[8];
} llk_schedule_entry;

/* loadScheduleDB + selectBest (ScheduleLoader.cpp:31-98,
 * ScheduleSelection.cpp:46-67): entries whose "operation" equals op_name and
 * whose shape.M_bucket equals m_bucket (shape.N and shape.K must be present
 * but are not compared), first match wins; with no match, the built-in
 * default {8,32,32,1,4,8,4,1,"n"}.  Returns LLK_OK, or LLK_ERR_NOT_FOUND
 * when the file cannot be read or parsed (out = default, like the
 * reference's warn-and-fall-back), and sets *n_matches. */
int llk_select_schedule(const char* db_path, const char* op_name,
                        int m_bucket, llk_schedule_entry* out, int* n_matches);

/* Makes `path` the active schedule DB of the dispatcher (NULL or "" clears
 * it; without a call, the file named by the LLK_SCHEDULE_DB environment
 * variable is used, if any).  For each (operation, M bucket) the entry the
 * loader above selects sets the launch: small-M kernel -> 32-column groups
 * per workgroup = BN / 32 (1, 2, 4) and k splits = grain_size; tile kernel
 * -> k splits = grain_size; grain_size 0 leaves the split count to the
 * shape heuristics.  Forced knobs (llk_set_tunable) take precedence.  This
 * is the reference's ScheduleSelection (ScheduleSelection.cpp:46-67)
 * driving the launch instead of the tiling pass.  LLK_ERR_NOT_FOUND when the
 * file cannot be read or parsed (the DB is then cleared). */
int llk_set_schedule_db(const char* path);

/* ----------------------------------------------------------------------- */
/* Synthetic inputs (no reference counterpart; used by llk-bench)          */
/* ----------------------------------------------------------------------- */

/* Fills HOST buffer out[0..n) with bf16 bits of sigma * N(0,1): counter-based
 * splitmix64 streams (s0 = seed ^ stream * 0x9E3779B97F4A7C15) and
 * Box-Muller, scaled in fp32 and rounded to nearest even.  threads <= 0 uses
 * every hardware thread.  Deterministic for a given (seed, stream, n). */
int llk_fill_normal_bf16(uint64_t seed, uint64_t stream, float sigma,
                         uint16_t* out, int64_t n, int threads);

/* ----------------------------------------------------------------------- */
/* Backend knobs (no reference counterpart)                                 */
/* ----------------------------------------------------------------------- */

/* Named integer knobs of the dispatch heuristics: "decode_max_m" (largest M
 * sent to the small-M kernel), "decode_splits" (force its k-split count,
 * 0 = cost model), "decode_target_wgs", "decode_min_kb",
 * "decode_group_width" (force the 32-column groups per small-M workgroup:
 * 1, 2, 4; 0 = cost model; a forced width runs the small-M kernel),
 * "decode_tile" (1: M <= 64 with K % 64 == 0 and 16-byte aligned X rows
 * runs on the decode tile kernel; 0: always the small-M kernel),
 * "midm_max_m" (largest M above 64, at most 256, that runs on the decode
 * tile kernel's 128- and 256-row forms when K % 64 == 0 and X rows are
 * 16-byte aligned; default 128; 64 or less: the tile kernels from M = 65 on),
 * "tile_splits" (force the tile kernel's k-split count, 0 = cost model),
 * "tile_wgs_per_wave", "tile_min_kb", "tile_tail_split" (1: the columns
 * of a partial last wave of tiles may run as a separate k-split launch;
 * 0: never; a forced "tile_splits" also turns it off), "tile_wide" (1:
 * the cost model may take the wide SwiGLU tiles; 0: never; 7 or 11: that
 * width), "kernel_fn_rowmajor" (1: the KernelFn entries -- SwiGLU and, from
 * the object-code level, matmul -- read device weights
 * with aligned rows straight into the kernels' row-major forms; 0: they
 * pack the weights on every call), "max_workspaces" (library-owned
 * workspaces kept per device, see llk_workspace_stats).
 * Returns LLK_OK or LLK_ERR_INVALID_ARGUMENT for an unknown name. */
int llk_set_tunable(const char* name, int64_t value);
int llk_get_tunable(const char* name, int64_t* value);

/* ----------------------------------------------------------------------- */
/* Serialized packed weights (the reference's L4 stores packed weights as   */
/* opaque blobs: JitCache.h:143-146; this is that blob's format, also used  */
/* on disk)                                                                 */
/* ----------------------------------------------------------------------- */

/* Blob: a 96-byte little-endian header
 *   magic "LLKPW950" | u32 version (1) | u32 dtype | i64 K | i64 N | i64 BK
 *   | i64 K_blocks | i64 block_size | i64 KB | i64 NB | u64 payload bytes
 *   | u64 FNV-1a 64 of the payload | u64 reserved (0)
 * followed by the device payload (MFMA operand order, llk_pack_device_layout).
 * llk_packed_weights_serialize writes it into `out` (capacity `cap`; with
 * out == NULL only *len is set); a device payload is copied back from the
 * GPU, a host-only handle's is computed on the host. */
int llk_packed_weights_serialize(const llk_packed_weights* pw, void* out, size_t cap,
                                 size_t* len);
/* Rebuilds a handle from a blob (header and checksum verified):
 * flags 0 -> device payload on the current device; LLK_PACK_KEEP_HOST ->
 * also the reference host layout; LLK_PACK_HOST_ONLY -> host layout only. */
int llk_packed_weights_deserialize(const void* blob, size_t len, unsigned flags,
                                   llk_packed_weights** out);
/* The same through a file. */
int llk_packed_weights_save(const llk_packed_weights* pw, const char* path);
int llk_packed_weights_load(const char* path, unsigned flags, llk_packed_weights** out);

/* ----------------------------------------------------------------------- */
/* Kernel / weight cache (JitCache: JitCache.h:67-218, JitCache.cpp:41-88,  */
/* 247-397)                                                                 */
/* ----------------------------------------------------------------------- */

/* KernelKey (KernelKey.h:45-57): same fields, types and order.  Enum values
 * as in the reference; this backend adds operation 3 (Matmul), layout 2
 * (the device payload order) and isa 7 (gfx950). */
typedef struct llk_kernel_key {
  uint8_t operation;     /* 0 FusedSwiGLU, 1 RoPE, 2 Attention, 3 Matmul */
  uint8_t input_type;    /* llk_dtype */
  uint8_t output_type;   /* llk_dtype */
  int64_t M_bucket;      /* 0-4 (llk_classify_m), -1 generic */
  int64_t N;
  int64_t K;
  uint8_t weight_layout; /* 0 RowMajor, 1 PackedKN, 2 device payload */
  uint8_t isa;           /* 0..6 CPU ISAs of the reference, 7 gfx950 */
  uint8_t math_mode;     /* 0 Strict, 1 BoundedFast, 2 UnsafeFast */
  uint16_t thread_count;
  uint64_t compiler_version;
  uint64_t schedule_version;
} llk_kernel_key;

/* WeightKey (KernelKey.h:114-124). */
typedef struct llk_weight_key {
  const void* weight_ptr;
  uint64_t shape_hash;
  int64_t BK;
  int64_t BN;
} llk_weight_key;

/* CacheStats (JitCache.h:67-71): index 0..3 = L1..L4. */
typedef struct llk_cache_stats {
  size_t hits[4];
  size_t misses[4];
  size_t evictions[4];
} llk_cache_stats;

/* MemRef2D (JitCache.h:43-51): the same seven fields in the same order (56
 * bytes).  Element strides; the data address is aligned + offset elements. */
typedef struct llk_memref2d {
  void* allocated;
  void* aligned;
  int64_t offset;
  int64_t size0;
  int64_t size1;
  int64_t stride0;
  int64_t stride1;
} llk_memref2d;

/* JitCache::KernelFn (JitCache.h:79-81): x, wg, wu, init, result.  No
 * return value: the calling thread's status of its last KernelFn call is
 * llk_kernel_fn_status(), its message llk_last_error(). */
typedef void (*llk_memref_kernel_fn)(llk_memref2d* x, llk_memref2d* wg, llk_memref2d* wu,
                                     llk_memref2d* init, llk_memref2d* result);

/* The other shape of an object-code entry: packed-weight handles, a
 * stream and a workspace, with llk_swiglu_bf16's signature (w1 is ignored
 * by matmul entries).  No reference counterpart. */
typedef int (*llk_kernel_fn)(const llk_tensor2d* x, const llk_packed_weights* w0,
                             const llk_packed_weights* w1, llk_tensor2d* y, int y_dtype,
                             llk_kernel_context* ctx);

typedef struct llk_jit_cache llk_jit_cache;

/* JitCache() / ~JitCache().  Destroying the cache frees the packed-weight
 * handles it owns (release acquired references first). */
int llk_cache_create(llk_jit_cache** out);
void llk_cache_destroy(llk_jit_cache* c);

/* lookupOrCompile(const KernelKey&, ModuleOp) (JitCache.h:107-109,
 * JitCache.cpp:247-250): the KernelFn of the key -- from L3, or on a miss
 * from the key's gfx950 code object, inserted into L3.  Code objects are
 * compiled ahead of time, one per operation (llk_fused_swiglu_gfx950.hsaco,
 * llk_matmul_gfx950.hsaco; see llk_code_object_path), so no module is
 * passed: on a miss the key's object is read and checked (64-bit AMDGPU
 * ELF, gfx950, defines kernels) and, when a HIP device is present, loaded
 * on the current device with hipModuleLoadData and its kernels resolved
 * with hipModuleGetFunction (else at the entry's first call on a device;
 * each device loads it once, and it stays loaded until the process ends).
 * The entry has the reference's KernelFn shape and behaviour -- that of
 * llk_swiglu_kernel_fn (below), result element type = the key's output
 * type -- but runs the kernels of the loaded code object, the pack kernel
 * included.  For a matmul key the entry computes result = init + x wg
 * (linalg.matmul's outs(init) semantics; wu is unused and may be NULL).
 * Errors: LLK_ERR_UNSUPPORTED_ARCH (isa != 7, or the object is not for
 * gfx950), LLK_ERR_DTYPE (input not bf16; output not bf16/f32, or f16 for
 * a matmul), LLK_ERR_INVALID_ARGUMENT (RoPE, Attention or an unknown
 * operation; N or K < 1; a file that is no code object), LLK_ERR_NOT_FOUND
 * (the key's code object is missing), LLK_ERR_HIP (the load failed).  On an
 * error nothing is inserted. */
int llk_cache_lookup_or_compile(llk_jit_cache* c, const llk_kernel_key* key,
                                llk_memref_kernel_fn* out);

/* The same L3 entry in its packed-handle shape (llk_kernel_fn), bound to
 * the key's output type (another y_dtype: LLK_ERR_DTYPE).  No reference
 * counterpart. */
int llk_cache_lookup_or_compile_packed(llk_jit_cache* c, const llk_kernel_key* key,
                                       llk_kernel_fn* out);

/* lookupOrCompile(const std::string& cache_key, ModuleOp) (JitCache.h:
 * 103-105, JitCache.cpp:182-245), the overload llk-compile calls with
 * "llk_" + hash(module) + "_M<M>_N<N>_K<K>" (llk-compile.cpp:298-310): the
 * L3 entry under `cache_key`, or on a miss the KernelFn of the module's
 * entry -- its first llk.fused_swiglu or llk.matmul op, in the reference's
 * MLIR text form (`module`, module_len bytes) -- with the op's result
 * element type, inserted under cache_key.  A module without such an op is
 * LLK_ERR_INVALID_ARGUMENT "No exported kernel entry point found in module"
 * (JitCache.cpp:214-220); other errors as llk_cache_lookup_or_compile. */
int llk_cache_lookup_or_compile_str(llk_jit_cache* c, const char* cache_key, const char* module,
                                    size_t module_len, llk_memref_kernel_fn* out);

/* Directory this cache reads code objects from (NULL or "": the default,
 * $LLK_CODE_OBJECT_DIR or else objects/ beside the library).  No
 * reference counterpart (the reference compiles in process). */
int llk_cache_set_object_dir(llk_jit_cache* c, const char* dir);

/* Path of the code object of `operation` (0 fused_swiglu, 3 matmul) in
 * `dir` (NULL or "": the default directory), written to buf (up to cap
 * bytes, NUL-terminated).  Returns its length, or LLK_ERR_INVALID_ARGUMENT
 * for an operation without one. */
int llk_code_object_path(int operation, const char* dir, char* buf, size_t cap);

/* Reads and checks the code object at `path` without loading it: LLK_OK
 * with its kernel count and newline-separated kernel symbols (up to cap
 * bytes, NUL-terminated; *len = full length), or LLK_ERR_NOT_FOUND,
 * LLK_ERR_INVALID_ARGUMENT (not an ELF code object, no kernels) or
 * LLK_ERR_UNSUPPORTED_ARCH (not AMDGPU gfx950). */
int llk_code_object_info(const char* path, int* kernel_count, char* names, size_t cap,
                         size_t* len);

/* L3 (JitCache.cpp:256-276), packed-handle shape: lookup returns 1 on a hit
 * (*out set), 0 on a miss; insert returns LLK_OK (a later
 * llk_cache_lookup_or_compile of the key adds the KernelFn shape). */
int llk_cache_lookup_object_code(llk_jit_cache* c, const llk_kernel_key* key, llk_kernel_fn* out);
int llk_cache_insert_object_code(llk_jit_cache* c, const llk_kernel_key* key, llk_kernel_fn fn);

/* L1 (level 1, IR) and L2 (level 2, optimized MLIR) string levels
 * (JitCache.cpp:282-310).  Lookup returns 1 on a hit and copies up to `cap`
 * bytes of the value into `out` (*len = full length), 0 on a miss. */
int llk_cache_insert_blob(llk_jit_cache* c, int level, const char* key, size_t key_len,
                          const void* value, size_t value_len);
int llk_cache_lookup_blob(llk_jit_cache* c, int level, const char* key, size_t key_len,
                          void* out, size_t cap, size_t* len);

/* L4 (JitCache.cpp:314-328), holding packed-weight handles instead of
 * blobs.  Insert transfers ownership of `pw` to the cache: a replaced or
 * evicted handle is freed once no acquired reference holds it; inserting
 * the handle its key already holds only refreshes the entry; a handle
 * belongs under one key at a time; on LLK_ERR_OUT_OF_MEMORY the handle has
 * been freed.  Lookup returns 1 with a borrowed handle, valid until the
 * entry is evicted or the cache is cleared or destroyed, or 0 on a miss. */
int llk_cache_insert_packed_weights(llk_jit_cache* c, const llk_weight_key* key,
                                    llk_packed_weights* pw);
int llk_cache_lookup_packed_weights(llk_jit_cache* c, const llk_weight_key* key,
                                    llk_packed_weights** out);
/* L4 lookup by (w->data, shape, bk), packing on a miss: from host memory
 * (llk_pack_weights, flags as there) or, with on_device != 0, from device
 * memory (llk_pack_weights_device on the default stream).  The WeightKey is
 * {w->data, hash of (K, N, stride0), bk, 128}.  One pack per key: callers
 * that miss on a key being packed wait for that pack and share its handle.
 * *out is borrowed as above. */
int llk_cache_get_packed_weights(llk_jit_cache* c, const llk_tensor2d* w, int64_t bk,
                                 int on_device, unsigned flags, llk_packed_weights** out);
/* llk_cache_get_packed_weights with a counted reference instead of a
 * borrowed handle (the reference's L4 hands out copies: JitCache.cpp:
 * 314-320): the handle stays valid, whatever eviction, replacement or
 * clear does to the level, until every acquire of it on this cache has
 * been matched by a release.  Release returns LLK_ERR_INVALID_ARGUMENT for
 * a handle with no reference held. */
int llk_cache_acquire_packed_weights(llk_jit_cache* c, const llk_tensor2d* w, int64_t bk,
                                     int on_device, unsigned flags, llk_packed_weights** out);
int llk_cache_release_packed_weights(llk_jit_cache* c, llk_packed_weights* pw);

/* evictLRU / setMaxEntries (JitCache.cpp:332-363): level 1..4; trims the
 * level to at most max_entries and makes that its capacity.  Returns
 * LLK_ERR_INVALID_ARGUMENT for another level (the reference ignores it). */
int llk_cache_evict_lru(llk_jit_cache* c, int level, size_t max_entries);
int llk_cache_set_max_entries(llk_jit_cache* c, int level, size_t max_entries);
/* getStats / clear / size (JitCache.cpp:365-397). */
int llk_cache_get_stats(const llk_jit_cache* c, llk_cache_stats* out);
void llk_cache_clear(llk_jit_cache* c);
size_t llk_cache_size(const llk_jit_cache* c);

/* ----------------------------------------------------------------------- */
/* The reference's KernelFn calling convention (JitCache.h:43-51, 79-81)    */
/* ----------------------------------------------------------------------- */

/* The fused SwiGLU with exactly the KernelFn shape, a drop-in for the
 * function JitCache::lookupOrCompile returns for an llk.fused_swiglu module
 * (JitCache.h:79-109): bf16 x [M, K], raw row-major bf16 wg, wu [K, N],
 * init and result [M, N] (callers pass init == result; init is only
 * shape-checked), result = bf16(SiLU(x wg) * (x wu)).  Like the JIT'd
 * function, every call reads wg and wu as they are at the call, so a caller
 * may rewrite a weight buffer in place or reuse its address between calls:
 * device-resident weights with 16-byte aligned rows (row stride a multiple
 * of 8) go straight to the kernels' row-major forms -- the decode tile
 * kernel's for at most 128 rows of X, the tile kernel's above (K a
 * multiple of 64, N of 8) -- and other weights are packed into the
 * MFMA operand layout on the device first (one pack launch per matrix into
 * a buffer the library owns per device).
 * Operands may be device memory (used in place) or host memory (staged
 * through device buffers).  Runs on the null stream and returns when the
 * result is written, like the reference's JIT'd function.  Calls on one
 * device from several threads are safe: they run one at a time.  No return
 * value: the status of the calling thread's last call is
 * llk_kernel_fn_status(), its message llk_last_error(). */
void llk_swiglu_kernel_fn(llk_memref2d* x, llk_memref2d* wg, llk_memref2d* wu,
                          llk_memref2d* init, llk_memref2d* result);
int llk_kernel_fn_status(void);

/* Opt-in reuse of packed weights by every KernelFn-shaped call of the
 * process (llk_swiglu_kernel_fn and the entries of
 * llk_cache_lookup_or_compile): with on != 0 the caller promises that a
 * weight buffer's contents never change while its address is in use, and
 * wg / wu are resolved through the L4 level of the current device's cache
 * (llk_kernel_fn_cache; WeightKey = address, shape, BK 64: JitCache.h:
 * 143-146, KernelKey.h:114-124) as counted references, packed on the first
 * call only.  A caller that then rewrites a buffer in place clears that
 * cache.  Returns the previous setting (0, the default: pack every call).
 * No reference counterpart. */
int llk_kernel_fn_assume_immutable_weights(int on);

/* The cache the KernelFn-shaped calls use on the current device under
 * llk_kernel_fn_assume_immutable_weights(1) (created on first use, owned by
 * the library; llk_cache_get_stats / llk_cache_clear apply), or NULL
 * without a device. */
llk_jit_cache* llk_kernel_fn_cache(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* LLK_ABI_H */
