/*
 * annc_hip.h -- C-ABI of the MI355X (gfx950) fused-operator library.
 *
 * Drop-in boundary for ANNC's fused-operator hot path.  Every symbol is
 * extern "C", takes plain pointers and sizes, and never throws.  Integer
 * status codes follow TensorFlow's error-code numbering (0 = OK,
 * 3 = INVALID_ARGUMENT, 8 = RESOURCE_EXHAUSTED, 13 = INTERNAL); the message
 * for the last failure on the calling thread is returned by
 * annc_hip_last_error().
 *
 * Pointer classes:
 *   - "any" pointers may be host memory or HIP device memory; the library
 *     inspects them (hipPointerGetAttributes) and stages host data through
 *     the device on a stream of its own, one per calling thread and device,
 *     synchronising before it returns.  This is the contract of the XLA-CPU
 *     custom calls and the TF CPU ops; concurrent callers on different
 *     threads never share a stream.
 *   - "device" pointers must be device memory; those entry points enqueue on
 *     the caller's stream (a hipStream_t passed as void*, NULL = HIP's null
 *     stream of the current device) and return without synchronising.  The
 *     library keeps scratch memory per stream, so calls on one stream must
 *     be issued from one thread at a time.
 */
#ifndef ANNC_HIP_H_
#define ANNC_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Status                                                                    */
/* ------------------------------------------------------------------------ */
enum {
  ANNC_OK = 0,
  ANNC_INVALID_ARGUMENT = 3,
  ANNC_RESOURCE_EXHAUSTED = 8,
  ANNC_INTERNAL = 13,
};

/* Message of the last failed call on this thread ("" when none). */
const char* annc_hip_last_error(void);

/* Library version string. */
const char* annc_hip_version(void);

/* Synchronises `stream` and returns ANNC_INVALID_ARGUMENT if any kernel
 * enqueued on it since the previous call met an out-of-range row id (those
 * rows contribute zero); clears the flag.  The reference leaves such ids
 * undefined (embedding_fused_sparse_segment_reduce.cc:92-110 reads them
 * unchecked). */
int annc_hip_stream_status(void* stream);

/* ------------------------------------------------------------------------ */
/* ANNC_FLAGS  (replaces annc::ANNCFlags / annc::get_annc_flags,             */
/*              annc/service/cpu/annc_flags.h:25-39, annc_flags.cc:10-130)   */
/* ------------------------------------------------------------------------ */
/* 1 if `name` is enabled in the process-wide flag set parsed once from the
 * ANNC_FLAGS environment variable (annc_flags.cc:85-93, 164-172). */
int annc_flag_enabled(const char* name);
/* Resets the process-wide flag set to its defaults and parses `flags` with
 * the ANNC_FLAGS grammar (annc_flags.cc:95-162).  NULL or "" keeps defaults. */
void annc_flags_reset(const char* flags);
/* Writes "name=0|1\n" lines for every stored flag (sorted) into buf; returns
 * the number of bytes needed (excluding the terminator). */
int64_t annc_flags_dump(char* buf, int64_t len);

/* ------------------------------------------------------------------------ */
/* Which HLO fragments become ANNC fusions / custom calls                    */
/* (replaces KDnnRewriter selection: annc/service/cpu/kdnn_rewriter.h:25-59,  */
/*  kdnn_rewriter.cc:8-69, gemm_rewriter.cc:13-134, graph_opt.cc:8-129).      */
/* Host-only; reads the process-wide ANNC_FLAGS set.                          */
/* ------------------------------------------------------------------------ */
enum {
  ANNC_HLO_OTHER = 0,
  ANNC_HLO_PARAMETER = 1,
  ANNC_HLO_CONSTANT = 2,
  ANNC_HLO_DOT = 3,
  ANNC_HLO_ADD = 4,
  ANNC_HLO_MAXIMUM = 5,
  ANNC_HLO_MULTIPLY = 6,
  ANNC_HLO_SELECT = 7,
  ANNC_HLO_BROADCAST = 8,
  ANNC_HLO_GATHER = 9,
  ANNC_HLO_CONVERT = 10,
  ANNC_HLO_AND = 11,
  ANNC_HLO_COMPARE = 12,
  ANNC_HLO_DIVIDE = 13,
  ANNC_HLO_RESHAPE = 14,
  ANNC_HLO_REDUCE = 15,
  ANNC_HLO_SLICE = 16,
  ANNC_HLO_REDUCE_WINDOW = 17,
};
enum { ANNC_DT_OTHER = 0, ANNC_DT_PRED = 1, ANNC_DT_S32 = 2, ANNC_DT_S64 = 3, ANNC_DT_F32 = 4 };
#define ANNC_HLO_MAX_RANK 8
#define ANNC_HLO_MAX_OPERANDS 8
#define ANNC_HLO_MAX_FUSED 16

/* One instruction of the fragment.  Users of a node are the nodes that list
 * it as an operand, in node-index order (XLA's users() order when nodes are
 * numbered in program order). */
typedef struct annc_hlo_node {
  int32_t opcode;                             /* ANNC_HLO_* */
  int32_t dtype;                              /* ANNC_DT_* of the result */
  int32_t rank;
  int32_t num_operands;
  int64_t dims[ANNC_HLO_MAX_RANK];
  int32_t minor_to_major[ANNC_HLO_MAX_RANK];  /* row-major: rank-1, ..., 0 */
  int32_t operands[ANNC_HLO_MAX_OPERANDS];    /* node indices */
  int32_t has_control_deps;
} annc_hlo_node;

typedef struct annc_hlo_rewrite {
  int32_t matched;     /* 0: no rewriter fired */
  char target[32];     /* custom-call target or fusion name: "__matmul_add_relu",
                          "__layout_matmul", "__pooling", "sparse_embedding2", ... */
  int32_t custom_call; /* 1: a custom call replaces the fusion; 0: fusion only */
  int32_t benefit;
  int32_t num_fused;
  int32_t fused[ANNC_HLO_MAX_FUSED];            /* fusion root first */
  int32_t num_operands;                         /* call operands before the shape infos */
  int32_t operands[2 * ANNC_HLO_MAX_OPERANDS];  /* node indices; -1 / -2 = the slice
                                                   starts / limits constants (__pooling) */
  int32_t num_shape_infos;                      /* then one s64[2*rank] get_param_info
                                                   constant per listed node */
  int32_t shape_info_of[2 * ANNC_HLO_MAX_OPERANDS];
} annc_hlo_rewrite;

/* Runs the rewriters that ANNC's visitor would run on nodes[instr]
 * (kDot: graph-opt + GEMM; kMultiply, kSelect: graph-opt), by descending
 * benefit (ties in registration order), and fills `out` for the first that
 * matches.  Returns ANNC_OK (out->matched tells whether one fired) or
 * ANNC_INVALID_ARGUMENT for a malformed fragment. */
int annc_hlo_rewrite_instruction(const annc_hlo_node* nodes, int64_t num_nodes, int32_t instr,
                                 annc_hlo_rewrite* out);

/* ------------------------------------------------------------------------ */
/* XLA-CPU custom-call targets (annc/service/cpu/kdnn_rewriter.h:140-155).    */
/* Same names, same operand order, same shape-info encoding                  */
/* (annc/service/hlo_util.h:14-21: s64[2*rank] = dims..., minor_to_major...). */
/* `out` and `in[*]` are "any" pointers; the call is synchronous.            */
/* ------------------------------------------------------------------------ */
/* gemm_rewriter.cc:161-185  in = {A f32[m,k], B f32[k,n], shape(A), shape(B)} */
void __matmul(void* out, const void** in);
/* gemm_rewriter.cc:218-247  in = {E f32[m,n], A, B, shape(E), shape(A), shape(B)} ; out = A.B + E */
void __matmul_add(void* out, const void** in);
/* gemm_rewriter.cc:249-281  in = {Z, E, A, B, shape(Z), shape(E), shape(A), shape(B)} ; out = max(A.B + E, 0) */
void __matmul_add_relu(void* out, const void** in);
/* gemm_rewriter.cc:187-216  in = {A f32[b,m,k], B f32[b,k,n], shape(A), shape(B)} */
void __batch_matmul(void* out, const void** in);
/* gemm_rewriter.cc:136-159  in = {A f32[m,k], Bpk (layout_matmul-packed [k,n]), shape(A), shape(B)} */
void __layout_matmul(void* out, const void** in);
/* graph_opt.cc:131-176  in = {ids s64[m,k], gathered f32[m,k,n], slice_starts s64[3],
 *                             slice_limits s64[3], shape(ids), shape(gathered)} ; out f32[m,n] */
void __pooling(void* out, void** in);
/* reduce_rewriter.cc:31-46 (registered by REGISTER_ALL_GEMM_KERNELS,
 * kdnn_rewriter.h:148-155; the rewriter that would emit it is disabled,
 * reduce_rewriter.cc:24-27)  in = {axis (read as f32, unused), x f32,
 * shape(axis), shape(x) s64 with m = [0], n = [1]} ; out f32[n]:
 * out[i] = (sum of |x[i*m + j]|, j < m) / m, the reference's cblas_sasum
 * over n consecutive runs of m values. */
void __reduce_mean(void* out, const void** in);

/* Function pointer of a custom-call target by its registered name, or NULL.
 * Equivalent of the lookup XLA performs after
 * XLA_CPU_REGISTER_CUSTOM_CALL_TARGET (kdnn_rewriter.h:148-155). */
void* annc_custom_call_target(const char* name);
/* Calls cb(name, fn, user) once per target, in the order of
 * REGISTER_ALL_GEMM_KERNELS (kdnn_rewriter.h:148-155); returns the number
 * of targets. */
int annc_register_custom_call_targets(void (*cb)(const char* name, void* fn, void* user),
                                      void* user);

/* ------------------------------------------------------------------------ */
/* layout_matmul pre-pack (replaces annc-opt FormageChange kn->kn4,          */
/* python/annc/optimize/data_pack.py:24-149, constant_folding.py:77-88).     */
/* The packed array has exactly k*n elements (annc-opt re-saves variables in */
/* their original shape, constant_folding.py:85), laid out in MFMA fragment  */
/* order for the gfx950 kernel; format tag "mfma_f32_32x32x2_k16".           */
/* ------------------------------------------------------------------------ */
const char* annc_layout_matmul_rhs_format(void);
/* Host pointers.  Returns ANNC_OK or ANNC_INVALID_ARGUMENT. */
int annc_layout_matmul_pack_rhs(int64_t k, int64_t n, const float* src_kn, float* dst_packed);
int annc_layout_matmul_unpack_rhs(int64_t k, int64_t n, const float* src_packed, float* dst_kn);
/* Device-side pack of a device-resident row-major [k,n] weight. */
int annc_hip_layout_matmul_pack_rhs(void* stream, int64_t k, int64_t n, const float* src_kn,
                                    float* dst_packed);

/* ------------------------------------------------------------------------ */
/* Device GEMM (engine behind __matmul* / __batch_matmul / __layout_matmul)  */
/*   C[z] = epi( A[z] . B[z] (+ E[z]) (+ bias) )   row-major, fp32 MFMA       */
/* b_packed = 1: B is in annc_layout_matmul_pack_rhs order (ldb ignored).    */
/* epilogue bits: ANNC_EPI_RELU = max(x, 0) as std::max(x, 0.f)              */
/* (gemm_rewriter.cc:278-280); ANNC_EPI_SIGMOID = 1/(1+exp(-x)).             */
/* addend (lde, stride_e) and bias (length n) may be NULL.  All device.      */
/* Workspace: row-major B whose rows are not 16-byte aligned (packed per     */
/* call) and small products with a long K (K split across workgroups) use a  */
/* workspace per stream and calling thread (threads that share a stream     */
/* interleave their launches), which the library allocates, or grows, on     */
/* first use.  An outgrown one is kept until the process ends, since a HIP   */
/* graph captured with it replays with its address; each growth at least    */
/* doubles it, so those kept add up to less than the live one.  A captured   */
/* graph uses the workspace on every replay: its replays and other calls of  */
/* the capturing thread on that stream must not overlap.                     */
/* It never allocates while the stream is being captured into a HIP graph:   */
/* such a call then takes a path without workspace (slower, same results to  */
/* the GEMM tolerance), or uses the workspace an earlier call left.          */
/* Tuning: the environment variable ANNC_GEMM_PIPE = "mi16" or "mi16w8"      */
/* runs one-batch packed GEMMs with K % 32 == 0 on 16x16 MFMA blocks          */
/* (v_mfma_f32_16x16x4f32) instead of the default 32x32 tiling.               */
/* ------------------------------------------------------------------------ */
enum { ANNC_EPI_NONE = 0, ANNC_EPI_RELU = 1, ANNC_EPI_SIGMOID = 2 };
int annc_hip_gemm(void* stream, int64_t batch, int64_t m, int64_t n, int64_t k,
                  const float* a, int64_t lda, int64_t stride_a,
                  const float* b, int64_t ldb, int64_t stride_b, int b_packed,
                  const float* addend, int64_t lde, int64_t stride_e,
                  const float* bias, int epilogue,
                  float* c, int64_t ldc, int64_t stride_c);

/* Tower tail in one kernel: the last hidden layer on a packed weight and the
 * N -> 1 scoring layer after it,
 *   h      = epi( A . B + bias )                       [m, n]
 *   out[i] = score_epi( sum_j h[i, j] * w_score[j] + bias_score[0] )
 * summed over j in a fixed order.  No single counterpart in the reference:
 * there the hidden layer is a __layout_matmul custom call with XLA's bias
 * and ReLU fusion (gemm_rewriter.cc:136-159), and the n -> 1 dot stays an
 * XLA dot (its N = 1 fails the >= 12 rule, gemm_rewriter.cc:29-38) with
 * bias and logistic fused by XLA.  Here neither h nor a second launch goes
 * through memory: hidden may be NULL; when given (ldh >= n), h is stored as
 * well.  Requirements: n = 64, 128 or 256; k a multiple of n, at most 2048;
 * B in annc_layout_matmul_pack_rhs order, 16-byte aligned; A rows 16-byte
 * aligned (lda % 4 == 0); w_score holds n floats; bias and bias_score may be
 * NULL.  Otherwise ANNC_INVALID_ARGUMENT, and nothing is launched.  All
 * device pointers. */
int annc_hip_dense_score(void* stream, int64_t m, int64_t n, int64_t k, const float* a,
                         int64_t lda, const float* b_packed, const float* bias, int epilogue,
                         const float* w_score, const float* bias_score, int score_epilogue,
                         float* hidden, int64_t ldh, float* out, int64_t ldo);

/* ------------------------------------------------------------------------ */
/* Embedding bags and segment reduction (all device pointers)                */
/* ------------------------------------------------------------------------ */
enum { ANNC_COMBINER_SUM = 0, ANNC_COMBINER_MEAN = 1 };

/* CSR embedding bag: out[b, :] = reduce_{j in [offsets[b], offsets[b+1])}
 * table[ids[j], :], summed per dim in j order starting from 0.0f; mean
 * multiplies by 1.0f/count and leaves empty bags at 0
 * (embedding_fused_sparse_segment_reduce.cc:87-151).  ids are int32
 * (ids_is_64 = 0) or int64.  out row stride ldo >= dim. */
int annc_hip_embedding_bag(void* stream, const float* table, int64_t rows, int64_t dim,
                           const void* ids, int ids_is_64, const int64_t* offsets,
                           int64_t num_bags, int combiner, float* out, int64_t ldo);

/* Segment reduction with arbitrary (unsorted) segment ids, the engine of
 * KPFusedSparseSegmentReduce: out[seg_ids[i*seg_stride], :] += data[indices[i], :]
 * in index order; out has `batch` rows (rows without ids stay 0).  Positions
 * whose segment id lies outside [0, batch) are skipped.  seg_sorted = 1
 * promises non-decreasing segment ids (TF's SparseSegment* contract, and the
 * order a SparseTensor's row indices have), which skips the stable sort by
 * segment; 0 makes no assumption. */
int annc_hip_segment_reduce(void* stream, const float* data, int64_t rows, int64_t dim,
                            const void* indices, int indices_is_64, const int64_t* seg_ids,
                            int64_t seg_stride, int64_t n, int combiner, int64_t batch,
                            float* out, int seg_sorted);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc): annc_hip_segment_reduce with the same arguments and results,
 * plus `status` (device int32, optional): bit 0 is OR-ed in when a row id
 * lies outside the data (the caller clears it; NULL discards the flag).
 * It calls no hipMalloc/hipFree: its workspace is a 16 MiB device array of
 * the library, one per GPU, held until the process ends.  Inputs that need
 * more workspace than that are rejected with ANNC_INVALID_ARGUMENT (sorted
 * ids need none; any order: the stable counting sort needs
 * 8 * ceil(n/1024) * batch + 4 * n bytes and more, up to 16384 segments; the
 * radix sort beyond that about 16 * n bytes).  Every call on a GPU uses that
 * GPU's one array, so calls that overlap on one GPU (two streams, two
 * threads) race and must be serialised by the caller. */
int annc_hip_segment_reduce_noalloc(void* stream, const float* data, int64_t rows, int64_t dim,
                                    const void* indices, int indices_is_64,
                                    const int64_t* seg_ids, int64_t seg_stride, int64_t n,
                                    int combiner, int64_t batch, float* out, int seg_sorted,
                                    int32_t* status);

/* sparse_embedding2 kLoop fusion (graph_opt.cc:8-41 with the bound checks of
 * bisheng-cpu/embedding_simplify.cc:62-81):
 * out[i,:] = table[valid ? ids[i] : fallback_row, :] * (float)valid,
 * valid = 0 <= ids[i] < rows. */
int annc_hip_sparse_embedding2(void* stream, const float* table, int64_t rows, int64_t dim,
                               const void* ids, int ids_is_64, int64_t n, int64_t fallback_row,
                               float* out);

/* __pooling on device pointers (graph_opt.cc:131-176).  shapes: ids [m,k],
 * gathered [m,k,n], out [m,n]. */
int annc_hip_pooling(void* stream, const int64_t* ids, const float* gathered, int64_t m,
                     int64_t k, int64_t n, const int64_t* slice_starts3,
                     const int64_t* slice_limits3, float* out);

/* Unique + gather, the engine of KPFusedGather: keys[i * key_stride] for
 * i < n are de-duplicated in order of first occurrence; unique[r] is the
 * r-th distinct key, indices[i] the rank of keys[i], out[r, :] =
 * table[unique[r], :] (a zero row, and the stream's status word set, for a
 * key outside [0, rows)).  unique and out must hold n keys / n rows; the
 * count U is written to the device int64 *num_unique.  n is at most 2^29
 * (INVALID_ARGUMENT beyond, before any launch).  All device pointers,
 * asynchronous on `stream`. */
int annc_hip_unique_gather(void* stream, const float* table, int64_t rows, int64_t dim,
                           const int64_t* keys, int64_t key_stride, int64_t n,
                           int64_t* num_unique, int64_t* unique, int32_t* indices, float* out);

/* ------------------------------------------------------------------------ */
/* Hashing: FarmHash Fingerprint64 (farmhashna::Hash64, google/farmhash as  */
/* pinned by TensorFlow 2.15) and StringToHashBucketFast semantics          */
/* bucket = Fingerprint64(bytes) % num_buckets (unsigned).                  */
/* Strings are given as bytes + offsets[n+1] (int64).  All device pointers. */
/* ------------------------------------------------------------------------ */
int annc_hip_fingerprint64(void* stream, const char* bytes, const int64_t* offsets, int64_t n,
                           int nul_terminated, uint64_t* out);
int annc_hip_hash_bucket_strings(void* stream, const char* bytes, const int64_t* offsets,
                                 int64_t n, int64_t num_buckets, int nul_terminated,
                                 int64_t* buckets);
/* AsString(int64) (decimal, '-' for negatives) fused with the hash. */
int annc_hip_hash_bucket_int64(void* stream, const int64_t* ids, int64_t n, int64_t num_buckets,
                               int64_t* buckets);

/* Multi-field hashed embedding bags (hash -> bucket -> gather -> pool):
 * for field f and sample b, bag (f,b) = ids[offsets[f*batch+b] .. offsets[f*batch+b+1]),
 * bucket = Fingerprint64(AsString(id)) % num_buckets[f], rows gathered from
 * tables[f] ([table_rows[f], dim], num_buckets[f] <= table_rows[f]) and
 * reduced with the segment-reduce order; written to
 * out[b, f*dim .. f*dim+dim) with row stride ldo.  tables/table_rows/
 * num_buckets are HOST arrays of num_fields entries (tables[f] are device
 * pointers); ids/offsets/out are device pointers.  buckets_out (device,
 * optional) receives the bucket id of every input id. */
int annc_hip_hashed_embedding_bags(void* stream, int64_t num_fields, int64_t batch, int64_t dim,
                                   const float* const* tables, const int64_t* table_rows,
                                   const int64_t* num_buckets, const int64_t* ids,
                                   const int64_t* offsets, int combiner, float* out, int64_t ldo,
                                   int64_t* buckets_out);

/* ------------------------------------------------------------------------ */
/* TensorFlow custom ops (TF is absent: one C entry per op, same inputs,    */
/* attrs and error messages).  "any" pointers, synchronous.                 */
/* ------------------------------------------------------------------------ */
/* KPFusedSparseSegmentReduce (annc/tensorflow/ops/embedding_fused_ops.cc:29-39,
 * kernels/embedding_fused_sparse_segment_reduce.cc:27-164).
 * Inputs: data f32 (data_rank, data_dims), indices int32|int64 [N],
 * slice_input int64 (slice_rank, slice_dims), begin int32[begin_elems],
 * begin_1 int32[begin_1_elems]; attr combiner (0 sum, 1 mean).
 * Phase 1 (output == NULL): validates and stores the output row count
 * (max segment id + 1) in *out_rows.  Phase 2: also writes output
 * [*out_rows, data_dims[1]] and the scalar slice_output.
 * Errors: the reference OP_REQUIRES messages verbatim. */
int annc_kp_fused_sparse_segment_reduce(const float* data, int data_rank, const int64_t* data_dims,
                                        const void* indices, int indices_is_64,
                                        int64_t num_indices, const int64_t* slice_input,
                                        int slice_rank, const int64_t* slice_dims,
                                        const int32_t* begin, int64_t begin_elems,
                                        const int32_t* begin_1, int64_t begin_1_elems,
                                        int combiner, int64_t* out_rows, float* output,
                                        int32_t* slice_output);

/* KPFusedSparseSegmentReduceNonzero (annc/tensorflow/ops/embedding_fused_ops.cc:41-51,
 * kernels/embedding_fused_sparse_segment_reduce_nonzero.cc:39-372).
 * Inputs: data f32 (data_rank 1 or 2, data_dims), indices int32|int64 [N],
 * slice_input int64 (slice_rank, slice_dims), begin int32[begin_elems]
 * (segment id = slice_input[i, begin[1]]); attr combiner (0 sum, 1 mean).
 * The segments are reduced as KPFusedSparseSegmentReduce does (rows in index
 * order, mean = sum * (1/count)) and the values != 0 are listed, segments in
 * order of first appearance, dims ascending.  output_shape int32: [max_seg+1]
 * for 1-D data, [max_seg+1, D] for 2-D.  Phase 1 (output_indices == NULL):
 * *num_nonzero = the number of listed values.  Phase 2: *num_nonzero holds
 * that count on entry and output_indices int32 [count, 1] (1-D: segment) or
 * [count, 2] (2-D: segment, dim) and output_nonzero f32[count] are written.
 * Phase 2 recomputes from its operands; it is refused (INVALID_ARGUMENT)
 * when their count differs from *num_nonzero.
 * Errors: the reference OP_REQUIRES messages verbatim; indices outside the
 * data rows are reported (the reference reads them unchecked). */
int annc_kp_fused_sparse_segment_reduce_nonzero(
    const float* data, int data_rank, const int64_t* data_dims, const void* indices,
    int indices_is_64, int64_t num_indices, const int64_t* slice_input, int slice_rank,
    const int64_t* slice_dims, const int32_t* begin, int64_t begin_elems, int combiner,
    int32_t* output_shape, int64_t* num_nonzero, int32_t* output_indices,
    float* output_nonzero);

/* KPFusedGather (annc/tensorflow/ops/embedding_fused_ops.cc:114-121,
 * kernels/embedding_fused_gather.cc:26-85).  Inputs: data f32 (data_rank,
 * data_dims), slice_input int64 (slice_rank, slice_dims), begin int32
 * [begin_elems]; the key column is begin[1].  Outputs: out_unique int64[U]
 * (the op's "out_shape": distinct keys in order of first occurrence),
 * out_indices int32[N], out_data f32[U, data_dims[1]].  *num_unique = U.
 * Output pointers may be NULL (e.g. a first call that only sizes them).
 * Errors: the reference messages verbatim, with ANNC_INTERNAL as the
 * reference's errors::Internal. */
int annc_kp_fused_gather(const float* data, int data_rank, const int64_t* data_dims,
                         const int64_t* slice_input, int slice_rank, const int64_t* slice_dims,
                         const int32_t* begin, int64_t begin_elems, int64_t* num_unique,
                         int64_t* out_unique, int32_t* out_indices, float* out_data);

/* KPFusedBatchMatMulAddSigmoid (annc/tensorflow/ops/embedding_fused_ops.cc:134-139,
 * kernels/fused_batchmatmul_add_sigmoid.cc): output[b,i,j] =
 * sigmoid(bias[b,i,j] + sum_k lhs[b,i,k] * rhs[(b,)k,j]) with lhs [batch,m,k],
 * rhs [k,n] or [batch,k,n], bias of rank <= 3 broadcast from the right.
 * "any" pointers, synchronous; errors are the reference messages
 * (ANNC_INVALID_ARGUMENT). */
int annc_kp_fused_batch_matmul_add_sigmoid(const float* lhs, int lhs_rank,
                                           const int64_t* lhs_dims, const float* rhs, int rhs_rank,
                                           const int64_t* rhs_dims, const float* bias,
                                           int bias_rank, const int64_t* bias_dims,
                                           float* output);

/* KPFusedEmbeddingWithHashBucket
 * (python/tensorflow/kernels/fused_embedding_with_hash_bucket.cc:15-83):
 * out[i,:] = weight[Fingerprint64(s_i) % num_buckets, :] for non-empty s_i,
 * zeros for empty s_i; combiner is accepted and ignored as in the reference.
 * num_buckets must not exceed weight rows (the reference reads past the
 * table otherwise). */
int annc_kp_fused_embedding_with_hash_bucket(const char* bytes, const int64_t* offsets,
                                             int64_t batch, const float* weight, int64_t rows,
                                             int64_t dim, int64_t num_buckets, int combiner,
                                             float* output);
/* KPFusedDnnEmbeddingWithHashBucket / KPFusedLinearEmbeddingWithHashBucket
 * (fused_dnn_embedding_with_hash_bucket.cc:10-62,
 *  fused_linear_embdedding_with_hash_bucket.cc:13-72): hash of the
 * NUL-terminated prefix, rows with bucket >= rows left at zero. */
int annc_kp_fused_dnn_embedding_with_hash_bucket(const char* bytes, const int64_t* offsets,
                                                 int64_t batch, const float* weight, int64_t rows,
                                                 int64_t dim, int64_t num_buckets, float* output);
int annc_kp_fused_linear_embedding_with_hash_bucket(const char* bytes, const int64_t* offsets,
                                                    int64_t batch, const float* weight,
                                                    int64_t rows, int64_t dim,
                                                    int64_t num_buckets, float* output);
/* KPFusedSparseEmbedding (fused_sparse_embedding.cc:10-87): outputs
 * indices int64[n,2], values int64[*num_values], empty_row_indicator
 * uint8[*num_values], dense_shape int64[2] = {n, 1}.  A non-empty string
 * whose bucket is 0 adds an index row but no value (reference behaviour);
 * the reference's out-of-range reads past *num_values are not reproduced. */
int annc_kp_fused_sparse_embedding(const char* bytes, const int64_t* offsets, int64_t n,
                                   int64_t num_buckets, int64_t* output_indices,
                                   int64_t* output_values, uint8_t* empty_row_indicator,
                                   int64_t* output_shape, int64_t* num_values);


#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* ANNC_HIP_H_ */
