/*
 * mdl_hip.h -- C ABI of the MI355X (gfx950) sparse-feature path.
 *
 * The library libmdl_hip.so implements, as hand-written HIP kernels, the
 * single-GPU sparse hot path of an MDL/RankMixer-style ranker:
 *
 *   raw int64 hashes --bucketize--> ids --lookup/pool--> per-feature slots
 *   upstream grads  --sort/unique/segment-reduce--> per-row grads
 *                   --row-wise Adagrad--> updated rows + accumulators
 *
 * Every pointer argument is a device address unless its comment says "host".
 * `stream` is a hipStream_t passed as void*; every kernel of a call runs on it
 * in order and no call synchronises the device.  All calls return MDL_OK (0)
 * or a negative MDL_ERR_* code; mdl_last_error() gives the message of the
 * calling thread's last failure.
 *
 * Reference interfaces (paths relative to the wcrmu/MDL source tree) are
 * named next to each entry point.
 */
#ifndef MDL_HIP_H
#define MDL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MDL_OK = 0,
  MDL_ERR_INVALID = -1,     /* bad argument (shape, dtype, alignment, size) */
  MDL_ERR_HIP = -2,         /* a HIP runtime call failed */
  MDL_ERR_WORKSPACE = -3,   /* workspace smaller than the *_workspace_bytes query */
  MDL_ERR_UNSUPPORTED = -4  /* legal input outside what this build implements */
};

enum { MDL_F32 = 0, MDL_BF16 = 1 };

/* Pooling of one feature's bags. NONE: every id is its own output row. */
enum { MDL_POOL_NONE = 0, MDL_POOL_SUM = 1, MDL_POOL_MEAN = 2 };

/* Feature flags. EXCLUDE_NULL is the "exclude" null policy: ids equal to 0
 * carry weight 0 in the pooled sum and in the mean's denominator
 * (src/model.py:554-557); without it ("include_as_padding") every id counts.
 * ROWS_BY_POSITION (pooled features only) pools rows that are already
 * embedded: the row of id slot i is weight row i - ids_begin, whatever the id,
 * and the ids only decide the null weights; this is _mean_pool_categorical_bag
 * on its `embedded` input (src/model.py:509-570).  Such features emit no sort
 * keys (sentinel) since they own no table. */
enum { MDL_FLAG_EXCLUDE_NULL = 1, MDL_FLAG_ROWS_BY_POSITION = 2, MDL_FLAG_IDS_FROM_OFFSETS = 4 };
/* IDS_FROM_OFFSETS: the feature's ids are [offsets[bag_base], offsets[bag_base
 * + nb]) of this call (nb = num_bags; 1 for an unpooled feature, whose ids
 * then occupy one pseudo-bag of the offsets array), and [ids_begin, ids_begin
 * + num_ids) is only a bound that range is clamped into.  A batch whose bag
 * lengths change then reuses the same descriptors and chunk plan: one scan
 * of its lengths places every feature on the device (the training step
 * encoder of src/model.py:3782-3890 serves any batch).  Forward chunks of an
 * unpooled feature past its range this call do nothing. */

enum { MDL_BUCKET_PRE_HASHED = 0, MDL_BUCKET_MOD = 1, MDL_BUCKET_NONE = 2 };
enum { MDL_TRUNCATE_HEAD = 0, MDL_TRUNCATE_TAIL = 1 };

/* Row-access classes of a feature or table: weight dtype x output/gradient
 * dtype x whether every row access is 16-byte aligned.  Kernels are
 * specialised per variant = class x lane width: a lane moves C elements of a
 * row, C = 1 for the unaligned classes and otherwise one 16-byte vector of the
 * weight type (4 fp32, 8 bf16) doubled up to 8 while four lanes do not cover
 * the row and the doubled C divides dim; variant = 3*class + log2(C/4).  The
 * calls taking a `classes` mask launch only the variants whose bit
 * (1 << variant) is set, 0 meaning all.  mdl_feature_classes and
 * mdl_table_classes compute the mask of a host descriptor array with the
 * kernels' own rule; a mask that misses a present variant skips its rows.
 * Rows of any width are reduced: a row wider than 64 lanes of C elements
 * cover (dim > 64 * C) is walked by one wave in column blocks of 64 * C.
 * MDL_CLASSES_UNSUPPORTED is reserved: mdl_table_classes never sets it, and
 * every backward call that reduces rows returns MDL_ERR_UNSUPPORTED for a
 * mask carrying it. */
#define MDL_CLASSES_UNSUPPORTED 0x80000000u
enum {
  MDL_CLASS_F32_VEC = 0, MDL_CLASS_F32 = 1, MDL_CLASS_BF16_VEC = 2,
  MDL_CLASS_BF16 = 3, MDL_CLASS_BF16_F32_VEC = 4, MDL_CLASS_BF16_F32 = 5
};

/* Sequence output order (src/model.py:3074-3100). */
enum { MDL_SEQ_OLDEST_TO_NEWEST = 0, MDL_SEQ_NEWEST_TO_OLDEST = 1 };

/*
 * One feature (lookup request) of a grouped call.  The array of descriptors
 * lives in device memory.  Features that alias one table (shared embeddings)
 * carry the same weight/state/row_base/table.
 *
 * Ids of feature f are ids[ids_begin, ids_begin + num_ids) (see
 * MDL_FLAG_IDS_FROM_OFFSETS for ranges set by the offsets).  A pooled feature
 * has num_bags bags whose bounds are offsets[bag_base .. bag_base+num_bags]
 * (absolute indices into ids, non-decreasing).  A MDL_POOL_NONE feature has
 * one output row per id and ignores bag_base/num_bags.
 *
 * Output row r of feature f is out + r*out_stride (elements of odtype); the
 * upstream gradient has the same layout at grad.  For the backward, output
 * row r of feature f is the sort payload payload_base + r.
 */
typedef struct mdl_feature {
  uint64_t weight;        /* table rows [num_rows, dim], row-major, contiguous */
  uint64_t state;         /* fp32 row-wise Adagrad accumulator [num_rows], 0 if unused */
  uint64_t out;           /* output row 0 */
  uint64_t grad;          /* upstream gradient row 0, 0 when no backward */
  int64_t num_rows;
  int64_t out_stride;     /* elements between consecutive output/gradient rows */
  int64_t row_base;       /* first sort key of the table: key = row_base + id */
  int64_t payload_base;   /* first sort payload of this feature's output rows */
  int64_t ids_begin;
  int64_t num_ids;
  int64_t bag_base;
  int64_t num_bags;
  int32_t dim;
  int32_t wdtype;         /* MDL_F32 / MDL_BF16: weight rows */
  int32_t odtype;         /* MDL_F32 / MDL_BF16: out and grad rows */
  int32_t pooling;        /* MDL_POOL_* */
  int32_t flags;          /* MDL_FLAG_* */
  int32_t padding_idx;    /* ids equal to it get no gradient (F.embedding padding_idx) */
  int32_t table;          /* index into the mdl_table array of the backward */
  int32_t reserved;
} mdl_feature;            /* 128 bytes */

/* A unit of forward work: bags [first, first+count) of one pooled feature, or
 * ids [first, first+count) (relative to ids_begin) of a MDL_POOL_NONE feature. */
typedef struct mdl_chunk {
  int32_t feature;
  int32_t count;
  int64_t first;
} mdl_chunk;              /* 16 bytes */

/*
 * One table of a grouped backward.  Sort keys of the table are
 * [row_base, row_base + num_rows); tables are ordered by row_base.
 * `feature` is the only feature reading the table, or -1 when several alias it.
 */
typedef struct mdl_table {
  uint64_t weight;
  uint64_t state;
  int64_t num_rows;
  int64_t row_base;
  int32_t dim;
  int32_t wdtype;
  int32_t feature;
  int32_t gdtype;         /* MDL_F32 / MDL_BF16: gradient rows of every feature reading it */
} mdl_table;              /* 48 bytes */

/* ---------------------------------------------------------------- misc --- */

const char* mdl_last_error(void);
int32_t mdl_abi_version(void);   /* 6 */

/* ------------------------------------------------------------ bucketing --- */

/*
 * out[i] = bucket of raw[i].  MDL_BUCKET_PRE_HASHED: (uint64(raw) & (B-1)) + 1
 * with B = num_buckets a power of two, null (valid[i]==0) -> 0, and a non-null 0
 * counted in *error_count when validate_nonzero (the id is still (0&(B-1))+1).
 * Replaces src/features.py:360-376 and the vectorised src/dataloader.py:8463-8493,
 * src/dataloader.py:10173-10186.
 * MDL_BUCKET_MOD: 1 + floormod(raw - 1, num_buckets - 1) (Python floor-mod),
 * null -> 0.  Replaces the id rule of src/benchmark.py:1246-1250.
 * valid may be NULL (all non-null).  error_count may be NULL.
 */
int mdl_bucketize(const int64_t* raw, const uint8_t* valid, int64_t n,
                  int64_t num_buckets, int32_t mode, int32_t validate_nonzero,
                  int64_t* out, int32_t* error_count, void* stream);

/*
 * List features to CSR bags: truncation, flattening and bucketing in one
 * call.  Replaces the Arrow path of src/dataloader.py:8565-8665
 * (_list_truncate_array: head keeps a row's first max_length elements, tail
 * its last; pc.list_value_length with nulls as 0; pc.list_flatten) followed
 * by the bucketing of src/dataloader.py:8463-8493 (see mdl_bucketize).
 *   in_offsets [rows+1]: row r holds raw[in_offsets[r] .. in_offsets[r+1])
 *                        (Arrow list offsets; any base);
 *   row_valid  [rows]  : 0 = null row, length 0 (may be NULL: all present),
 *                        except under tail truncation, which follows the
 *                        reference in reading the raw offsets of every row
 *                        (src/dataloader.py:8583-8604): a null row keeps the
 *                        last max_length elements of its span;
 *   raw, elem_valid [n_in]: element values and validity (elem_valid may be
 *                        NULL); a null element keeps its slot and buckets to 0;
 *   max_length < 0     : no truncation; truncation MDL_TRUNCATE_HEAD / _TAIL;
 *   bucket_mode        : MDL_BUCKET_PRE_HASHED / MDL_BUCKET_MOD as in
 *                        mdl_bucketize, or MDL_BUCKET_NONE (values copied,
 *                        nulls 0; num_buckets unused).
 * Writes lengths [rows] (the kept counts), out_offsets [rows+1] (their
 * exclusive scan; the kept total is out_offsets[rows], in device memory) and
 * values[j] for j < values_capacity: the bucketed kept elements in row order,
 * zeros past the total (values_capacity = n_in always suffices; a smaller one
 * keeps the first values_capacity).  Row offsets outside [0, n_in] or
 * decreasing are clamped and counted in *error_count, as are non-null zeros
 * under pre_hashed with validate_nonzero (error_count may be NULL).
 * Nothing is read back to the host.
 */
size_t mdl_bag_truncate_workspace_bytes(int64_t rows);
int mdl_bag_truncate(const int64_t* in_offsets, const uint8_t* row_valid, int64_t rows,
                     const int64_t* raw, const uint8_t* elem_valid, int64_t n_in,
                     int64_t max_length, int32_t truncation, int32_t bucket_mode,
                     int64_t num_buckets, int32_t validate_nonzero, int64_t* lengths,
                     int64_t* out_offsets, int64_t* values, int64_t values_capacity,
                     int32_t* error_count, void* workspace, size_t workspace_bytes,
                     void* stream);

/* --------------------------------------------------------------- offsets --- */

/* offsets[0] = 0, offsets[i+1] = offsets[i] + lengths[i]; n+1 outputs.
 * Replaces the segment layout of repeat_interleave(arange(B), lengths) in
 * src/model.py:560-563,666-669 (CSR values+lengths, src/dataloader.py:8607-8665). */
size_t mdl_offsets_workspace_bytes(int64_t n);
int mdl_lengths_to_offsets(const int64_t* lengths, int64_t n, int64_t* offsets,
                           void* workspace, size_t workspace_bytes, void* stream);

/* -------------------------------------------------------------- planning --- */

/* Host helpers: variant masks (see MDL_CLASS_*) of host descriptor arrays. */
uint32_t mdl_feature_classes(const mdl_feature* feats_host, int32_t num_features);
uint32_t mdl_table_classes(const mdl_table* tables_host, int32_t num_tables);

/* Host helper: split every feature into forward chunks of about target_ids ids.
 * feats_host: host copy of the descriptors.  Writes at most `capacity`
 * chunks to chunks_host (host, may be NULL) and returns the number needed,
 * or a negative MDL_ERR_* code. */
int64_t mdl_plan_chunks(const mdl_feature* feats_host, int32_t num_features,
                        int32_t target_ids, mdl_chunk* chunks_host, int64_t capacity);

/* ------------------------------------------------------------- forward --- */

/*
 * Grouped lookup + pooling of every chunk, one launch for all features.
 *   MDL_POOL_NONE : out row r = weight[ids[ids_begin + r]]      (F.embedding,
 *                   src/embeddings.py:438-473, grouped :1646-1709)
 *   MDL_POOL_SUM  : out row b = sum_i w_i * weight[id_i]      (embedding_bag sum)
 *   MDL_POOL_MEAN : out row b = sum_i w_i * weight[id_i] / max(sum_i w_i, 1)
 *                   (src/model.py:509-570, batched :590-678)
 * with w_i = 0 for id 0 under MDL_FLAG_EXCLUDE_NULL and 1 otherwise; sums in
 * fp32, one rounding to odtype.  Empty bags give 0.  Ids outside
 * [0, num_rows) contribute 0 and are counted in *error_count (may be NULL);
 * so are bag offsets outside the feature's id range (clamped into it),
 * decreasing bag offsets and pooled chunks of more than 256 bags (skipped).
 * Under MDL_FLAG_ROWS_BY_POSITION, weight[id_i] reads weight[i - ids_begin].
 *
 * When sort_keys is not NULL the call also writes, for every id position i of
 * every feature, the backward sort key and payload:
 *   sort_keys[i]    = row_base + id, or `sentinel` when id is padding_idx,
 *                     invalid, or 0 under MDL_FLAG_EXCLUDE_NULL (no gradient
 *                     reaches it);
 *   sort_payload[i] = payload_base + output row of the id.
 * and, when bag_count is not NULL, bag_count[payload_base + b] = sum_i w_i for
 * every pooled bag.  sort_keys/sort_payload have one entry per position of
 * the concatenated ids array.  num_ids is the number of entries of ids: every
 * feature's id range is clamped into [0, num_ids), so a descriptor or bag
 * lengths that point past the array read nothing outside it (the clamp is
 * counted as an error).
 *
 * key_origin (device, may be NULL): position o = *key_origin (clamped into
 * [0, num_ids]) becomes entry 0 of sort_keys/sort_payload, i.e. position i is
 * written to entry i - o, and every feature's id range is clamped into
 * [o, num_ids).  A plan cut into key groups (rows of 2^32 - 1 or more) looks
 * up one group per call, with that group's first offset as the origin, so each
 * group's keys start at entry 0 of its own arrays even when the device alone
 * knows where its ids begin.  NULL: o = 0.
 */
int mdl_forward(const mdl_feature* feats, int32_t num_features,
                const mdl_chunk* chunks, int64_t num_chunks,
                const int64_t* ids, int64_t num_ids, const int64_t* offsets,
                uint32_t* sort_keys, uint32_t* sort_payload,
                const int64_t* key_origin, uint32_t sentinel,
                float* bag_count, int32_t* error_count, uint32_t classes,
                void* stream);

/*
 * Backward of bag pooling with respect to the pooled rows (the autograd of
 * src/model.py:564-570 and :672-676): for every id position i of a pooled
 * feature, in bag b,
 *   weight[i - ids_begin] = out[b] * w_i / max(bag_count[payload_base + b], 1)  (MEAN)
 *   weight[i - ids_begin] = out[b] * w_i                                         (SUM)
 * computed in fp32 and rounded once.  In this call `out` is read (the
 * upstream gradient of the pooled rows, odtype, row stride out_stride) and
 * `weight` is written ([num_ids, dim], wdtype): the per-position gradient of
 * the rows the forward pooled, i.e. the gradient of the `embedded` input of a
 * MDL_FLAG_ROWS_BY_POSITION feature, or the uncoalesced COO values of the
 * sparse embedding backward of a lookup feature.  Null weights w_i follow the
 * forward (ids, flags and num_rows as the forward had them); bag_count
 * (required) is what mdl_forward wrote
 * for these features.  chunks come from mdl_plan_chunks over
 * these descriptors and classes from mdl_feature_classes of them (0: all).
 * MDL_POOL_NONE features are skipped.
 */
int mdl_pool_backward(const mdl_feature* feats, int32_t num_features,
                      const mdl_chunk* chunks, int64_t num_chunks,
                      const int64_t* ids, int64_t num_ids, const int64_t* offsets,
                      const float* bag_count, uint32_t classes, void* stream);

/*
 * Sequence gather without pooling, right-aligned into a padded window
 * (src/model.py:3022-3072, alignment :2989-3020, order :3074-3100).
 * ids: [batch, in_len] right-padded; lengths: [batch].
 * out: [batch, out_len, dim] (odtype); mask: [batch, out_len] bytes.
 * Row b has len_b = clamp(lengths[b], 0, out_len) window entries (none when
 * in_len == 0); entry rel of row b sits at position p = out_len - len_b + rel
 * (mask 1) and holds weight[ids[b, src]] with src = min(rel, in_len - 1)
 * (oldest_to_newest) or min(len_b - 1 - rel, in_len - 1) (newest_to_oldest):
 * a length past the input width repeats the last input element, as the
 * reference's clamp of the source position does (:3011-3016).  Other
 * positions hold 0 (mask 0).
 * feature->out is ignored (out is passed here); feature->payload_base and
 * row_base are used when sort_keys is not NULL: for window entry (b, rel),
 * sort_keys[rel + b*out_len] = row_base + id (sentinel when rel >= len_b or
 * padding), payload = payload_base + b*out_len + p, so the key arrays hold
 * batch*out_len entries.  With key_offsets (device int64 [batch + 1],
 * nondecreasing; NULL for the dense layout above) the keys are packed: entry
 * rel < cap_b = key_offsets[b+1] - key_offsets[b] (at most out_len) of row b
 * goes to key_offsets[b] + rel and nothing is written past the cap, so a
 * backward over the key_offsets[batch] packed entries sorts no padding.
 * With cap_b = len_b every window entry is kept; a row longer than its cap
 * loses the rest, a shorter one pads its cap with sentinels.
 */
int mdl_sequence_forward(const mdl_feature* feature_host, const int64_t* ids,
                         const int64_t* lengths, int64_t batch, int64_t in_len,
                         int64_t out_len, int32_t order, void* out, uint8_t* mask,
                         uint32_t* sort_keys, uint32_t* sort_payload,
                         const int64_t* key_offsets, uint32_t sentinel,
                         int32_t* error_count, void* stream);

/* ---------------------------------------------------------------- sort --- */

/*
 * Stable LSD radix sort of (key, payload) pairs on the low key_bits bits,
 * 8 bits per pass, ping-ponging between (keys, payload) and (keys_alt,
 * payload_alt).  *result_in_alt (host) is set to 1 when the sorted pairs end
 * in the _alt buffers.  Equal keys keep input order, so the segment reduction
 * that follows sums duplicates in a fixed order (deterministic), unlike the
 * fp32-atomic index_add_ of the reference (src/optim.py:321-324 coalesce).
 */
size_t mdl_sort_workspace_bytes(int64_t n);
int mdl_sort_pairs(uint32_t* keys, uint32_t* payload, uint32_t* keys_alt,
                   uint32_t* payload_alt, int64_t n, int32_t key_bits,
                   void* workspace, size_t workspace_bytes, int32_t* result_in_alt,
                   void* stream);

/* torch.unique(sorted=True, return_inverse=True, return_counts=True) of
 * ids in [0, 2^key_bits): unique_out[U], inverse_out[n], counts_out[U] (counts
 * may be NULL), *num_unique written to device memory.  Replaces the
 * world>1 dedup of src/embeddings.py:514-519,549-553. */
size_t mdl_unique_workspace_bytes(int64_t n);
int mdl_unique(const int64_t* ids, int64_t n, int32_t key_bits, int64_t* unique_out,
               int64_t* inverse_out, int64_t* counts_out, int64_t* num_unique,
               void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------ backward --- */

/*
 * The backward of a grouped call consumes the sort keys/payloads written by
 * mdl_forward / mdl_sequence_forward (n entries, keys < 2^key_bits; the
 * sentinel must be < 2^key_bits too).  The calls that sort (sort, adagrad,
 * count) take `count`: NULL, or a device int64 holding how many of the n
 * entries are present this call (clamped to [0, n]) -- e.g. the last offset
 * of the forward's offsets scan -- so a batch whose size is only known on the
 * device is sorted and reduced without a host round trip; n is then the
 * capacity that sizes the launches and the workspace.  The calls that follow
 * a sort (apply, sumsq, coalesce) take the same n and read the rest of the
 * plan from the workspace.  It sorts them in place (keys/payload
 * and the workspace are clobbered), cuts the sorted array into chunks of
 * <= 512 entries that never straddle two tables and reduces every run of
 * equal keys.  The num_tables tables (device array) are ordered by row_base,
 * cover every non-sentinel key, and their gradients are 16-byte aligned with
 * row strides that are multiples of 16 bytes whenever dim*sizeof(weight) is.
 * dim <= 64*C (C the table's lane width above; 512 when dim is a multiple
 * of 8) and max_dim >= every dim.
 * The per-id gradient of a pooled id is grad[row b] / max(bag_count, 1) (mean)
 * or grad[row b] (sum, none); padding ids get none (src/model.py:564-570 and
 * the F.embedding sparse backward).  Duplicate ids are summed in input order
 * in fp32, deterministically.
 */
size_t mdl_backward_workspace_bytes(int64_t n, int32_t num_tables, int32_t max_dim);

/*
 * Sort keys/payloads of a plain row-index list, for coalescing an uncoalesced
 * COO gradient (indices [n], values [n, dim]) with the calls below as one
 * MDL_POOL_NONE feature whose gradient rows are the values
 * (sparse coalesce of src/optim.py:323-324, src/train.py:5388-5396):
 * keys[i] = row_base + ids[i] (sentinel when ids[i] == padding_idx, pass -1
 * for none, or outside [0, num_rows), counted in *error_count),
 * payload[i] = payload_base + i.
 */
int mdl_sparse_keys(const int64_t* ids, int64_t n, int64_t num_rows, int64_t row_base,
                    int64_t payload_base, int64_t padding_idx, uint32_t* keys,
                    uint32_t* payload, uint32_t sentinel, int32_t* error_count,
                    void* stream);

/*
 * Fused backward + row-wise Adagrad: every distinct (table, row) is updated
 * once from its summed gradient g (times *grad_scale when grad_scale, a
 * device float, is not NULL):
 *   acc += sum(g^2)/dim;  w = w - lr * (g / (sqrt(acc) + eps))
 * rounded once to the weight dtype (round-to-nearest-even for bf16).
 * Semantics of src/optim.py:31-62 (Triton kernel) and :299-357 (step); the
 * scale is the clip coefficient of src/train.py:5788-5826 applied to the
 * coalesced gradient before the step.
 */
int mdl_backward_adagrad(const mdl_feature* feats, int32_t num_features,
                         const mdl_table* tables, int32_t num_tables, int32_t max_dim,
                         uint32_t* sort_keys, uint32_t* sort_payload, int64_t n,
                         const int64_t* count, int32_t key_bits, const float* bag_count, float lr, float eps,
                         const float* grad_scale, void* workspace, size_t workspace_bytes,
                         uint32_t classes, void* stream);

/* mdl_backward_adagrad in two calls with the same arguments and workspace:
 * mdl_backward_sort (radix sort + chunk plan), then mdl_backward_apply
 * (segment reduction + update).  key_bits must be the sort's: the later
 * calls find the sorted pairs where its pass count left them.  (Keys wider
 * than key_bits are left unsorted; a reduce then touches no weight row or
 * accumulator for a key outside its chunk's table, and the result is wrong
 * but every access stays in bounds.) */
int mdl_backward_sort(const mdl_table* tables, int32_t num_tables, int32_t max_dim,
                      uint32_t* sort_keys, uint32_t* sort_payload, int64_t n,
                      const int64_t* count, int32_t key_bits, void* workspace, size_t workspace_bytes,
                      void* stream);
int mdl_backward_apply(const mdl_feature* feats, int32_t num_features,
                       const mdl_table* tables, int32_t num_tables, int32_t max_dim,
                       uint32_t* sort_keys, uint32_t* sort_payload, int64_t n,
                       int32_t key_bits, const float* bag_count, float lr, float eps,
                       const float* grad_scale, void* workspace, size_t workspace_bytes,
                       uint32_t classes, void* stream);

/*
 * Squared 2-norm of the coalesced gradient of every table,
 *   *sumsq = sum over distinct (table, row) of sum_j g[row, j]^2,
 * after mdl_backward_sort and with the same arguments and workspace (the
 * sorted pairs are kept, so mdl_backward_apply can follow).  With
 * mdl_clip_coef this fuses the sparse clip (src/train.py:5788-5826) into the
 * backward without materialising the coalesced gradient: sort, sumsq,
 * clip_coef, apply(grad_scale = coef).  Deterministic (fixed-order sums).
 */
int mdl_backward_sumsq(const mdl_feature* feats, int32_t num_features,
                       const mdl_table* tables, int32_t num_tables, int32_t max_dim,
                       uint32_t* sort_keys, uint32_t* sort_payload, int64_t n,
                       int32_t key_bits, const float* bag_count, float* sumsq,
                       void* workspace, size_t workspace_bytes, uint32_t classes,
                       void* stream);

/*
 * Coalesced sparse gradients, the autograd contract of src/optim.py:317-329 and
 * src/train.py:5730-5742 (rows ascending and unique), in two calls:
 * mdl_backward_count sorts and writes unique_range[2t], unique_range[2t+1]
 * (device int64), the global distinct-row index range of table t, so
 * U_t = unique_range[2t+1] - unique_range[2t];  mdl_backward_coalesce, with the
 * same keys/payload/key_bits/workspace, then writes rows (int64 [U_t]) and
 * values ([U_t, dim], weight dtype) at the device addresses rows_addr[t] and
 * values_addr[t] (device arrays of num_tables addresses).
 */
int mdl_backward_count(const mdl_table* tables, int32_t num_tables, int32_t max_dim,
                       uint32_t* sort_keys, uint32_t* sort_payload, int64_t n,
                       const int64_t* count, int32_t key_bits, int64_t* unique_range,
                       void* workspace, size_t workspace_bytes, void* stream);
int mdl_backward_coalesce(const mdl_feature* feats, int32_t num_features,
                          const mdl_table* tables, int32_t num_tables, int32_t max_dim,
                          uint32_t* sort_keys, uint32_t* sort_payload, int64_t n,
                          int32_t key_bits, const float* bag_count,
                          const int64_t* unique_range, const uint64_t* rows_addr,
                          const uint64_t* values_addr, void* workspace,
                          size_t workspace_bytes, uint32_t classes, void* stream);

/*
 * mdl_backward_adagrad without a workspace argument and without allocating:
 * no counterpart in the reference.  It is for callers that cannot allocate
 * device memory -- code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  Its scratch is a static device array of
 * mdl_noalloc_scratch_bytes() (64 MiB) per GPU, held until the process ends;
 * a call whose mdl_backward_workspace_bytes(n, num_tables, max_dim) exceeds
 * it returns MDL_ERR_UNSUPPORTED (e.g. 1 M entries over 1024 tables of
 * max_dim 128 need 45 MiB).  Every call on one GPU shares that GPU's array
 * and leaves its contents behind (the call initialises what it reads), so
 * calls that overlap on one GPU -- on different streams or host threads --
 * race.  The scratch used is the current device's: a non-null stream must
 * belong to the current device, else the call returns MDL_ERR_INVALID.
 * Otherwise the same arguments and results as mdl_backward_adagrad.
 */
size_t mdl_noalloc_scratch_bytes(void);
int mdl_backward_adagrad_noalloc(const mdl_feature* feats, int32_t num_features,
                                 const mdl_table* tables, int32_t num_tables, int32_t max_dim,
                                 uint32_t* sort_keys, uint32_t* sort_payload, int64_t n,
                                 const int64_t* count, int32_t key_bits, const float* bag_count,
                                 float lr, float eps, const float* grad_scale, uint32_t classes,
                                 void* stream);

/*
 * Capacity-sized coalesced gradients without a host read: after
 * mdl_backward_coalesce wrote table t's U_t unique rows and values at
 * rows_addr[t] / values_addr[t] (buffers of capacity[t] >= U_t entries,
 * capacity a device int64 [num_tables]), fill entries [U_t, capacity[t])
 * with the table's last unique row (row 0 when U_t = 0) and zero values
 * (dim elements of the table's dtype, rows contiguous).  The buffers are then
 * an uncoalesced COO gradient with the coalesced gradient's sum and a size
 * the host knows without waiting for the device (a table's id count bounds
 * U_t).  unit_first (device int64 [num_tables + 1]) is the prefix of
 * ceil(capacity[t] / 64) and units its last entry.
 */
int mdl_backward_pad(const mdl_table* tables, int32_t num_tables, const int64_t* unique_range,
                     const uint64_t* rows_addr, const uint64_t* values_addr, const int64_t* capacity,
                     const int64_t* unit_first, int64_t units, void* stream);

/* ------------------------------------------------------------ clipping --- */

/* A contiguous gradient tensor (dense, or the values of a coalesced COO).
 * With live_rows set, only the first min(numel, *live_rows * row_elems)
 * elements count: the live rows of a capacity-sized sparse gradient, whose
 * row count is known on the device only.  The sum of squares cuts a span
 * into slices by that live element count, so a capacity-sized gradient and
 * its exact coalesced counterpart give the same bits. */
typedef struct mdl_span {
  uint64_t data;          /* device address */
  int64_t numel;
  int32_t dtype;          /* MDL_F32 / MDL_BF16 */
  int32_t row_elems;      /* elements per row (with live_rows) */
  const int64_t* live_rows; /* device int64, or NULL: all numel elements */
} mdl_span;               /* 32 bytes */

/*
 * Sparse gradient clipping of the trainer (_clip_sparse_grad_norm,
 * src/train.py:5788-5826, with _gradient_squared_norm :5745-5753 and
 * _scale_gradients :5756-5772), as three stream-ordered calls that never
 * synchronise:
 *   mdl_sumsq      *sumsq = sum over spans of sum_i x_i^2 (fp32 squares and
 *                  partials, fp64 final sum; deterministic).  spans: device
 *                  array of num_spans (<= 65535) descriptors.
 *   mdl_clip_coef  total = sqrt(sumsq[0] + ... + sumsq[count-1]) (fp32, in
 *                  order), *total_norm = total (may be NULL),
 *                  *coef = min(max_norm / (total + 1e-6), 1).
 *   mdl_scale      x *= *coef in place, in each span's dtype (bf16: the
 *                  coefficient rounded to bf16, one rounding of the product).
 */
size_t mdl_sumsq_workspace_bytes(int32_t num_spans);
int mdl_sumsq(const mdl_span* spans, int32_t num_spans, float* sumsq,
              void* workspace, size_t workspace_bytes, void* stream);
int mdl_clip_coef(const float* sumsq, int32_t count, float max_norm,
                  float* total_norm, float* coef, void* stream);
int mdl_scale(const mdl_span* spans, int32_t num_spans, const float* coef, void* stream);

/* ------------------------------------------------------------- update --- */

/*
 * Row-wise Adagrad on unique rows of one table (fused_rowwise_adagrad_update,
 * src/optim.py:68-108, kernel :31-62): for every i,
 *   acc[rows[i]] += sum_j values[i,j]^2 / dim
 *   weight[rows[i]] = weight[rows[i]] - lr * values[i] / (sqrt(acc) + eps).
 * rows must be unique and inside [0, num_rows) (rows outside are skipped and
 * counted in *error_count, may be NULL).  values_stride in elements.
 */
int mdl_rowwise_adagrad(void* weight, int32_t wdtype, int64_t num_rows, int32_t dim,
                        int64_t weight_stride, float* acc, const int64_t* rows,
                        int64_t num_touched, const void* values, int32_t vdtype,
                        int64_t values_stride, float lr, float eps,
                        int32_t* error_count, void* stream);

/*
 * One table of a grouped row-wise Adagrad step.  rows[0 .. n) are the unique
 * touched rows (int64) and values[i] their gradient rows (vdtype, stride
 * values_stride elements), n = *count (device int64; count = 0 means n =
 * capacity).  unit_first is the prefix, over the tables before this one, of
 * ceil(capacity / MDL_UPDATE_UNIT) -- the host fills it.
 */
typedef struct mdl_update {
  uint64_t weight;        /* [num_rows, dim], row stride weight_stride elements */
  uint64_t state;         /* fp32 accumulator [num_rows] */
  uint64_t rows;
  uint64_t values;
  uint64_t count;         /* device int64 address, or 0 */
  int64_t num_rows;
  int64_t capacity;
  int64_t weight_stride;
  int64_t values_stride;
  int64_t unit_first;
  int32_t dim;
  int32_t wdtype;
  int32_t vdtype;
  float lr;               /* this table's learning rate (per-parameter decay) */
} mdl_update;             /* 96 bytes */

#define MDL_UPDATE_UNIT 256

/*
 * Row-wise Adagrad of every table of an optimizer step in one launch: for
 * each table and each i < n, the update of mdl_rowwise_adagrad with the
 * table's lr (ShardedRowWiseAdagrad.step, src/optim.py:299-377, which makes
 * one fused_rowwise_adagrad_update launch per parameter, :68-108).  updates
 * is the device array, updates_host a host copy (validated, and used to pick
 * the kernels); n comes from device memory, so a gradient whose row count is
 * only known on the device (capacity-sized, see mdl_backward_pad) needs no
 * host read.  Rows outside [0, num_rows) are skipped and counted.
 */
uint32_t mdl_update_classes(const mdl_update* updates_host, int32_t num_updates);
int mdl_grouped_rowwise_adagrad(const mdl_update* updates, const mdl_update* updates_host,
                                int32_t num_updates, float eps, int32_t* error_count, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MDL_HIP_H */
