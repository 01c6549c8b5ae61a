/*
 * cu_roaring_abi.h -- the C-ABI boundary of the MI355X Roaring library.
 *
 * Plain C: pointers, sizes and status codes only.  Every entry point returns
 * CR_OK (0) on success or a CR_ERR_* code; cr_last_error() returns a
 * thread-local message for the last failure on the calling thread.  Device
 * pointers are HIP device pointers; `stream` is a hipStream_t (NULL = the
 * default stream).  Producing calls are stream-ordered and synchronise
 * `stream` once before returning, so every host-side field of the returned
 * struct is valid on return (the reference's contract).
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the reference checkout).
 */
#ifndef CU_ROARING_ABI_H
#define CU_ROARING_ABI_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CR_OK 0
#define CR_ERR_HIP 1          /* a HIP runtime call failed */
#define CR_ERR_INVALID 2      /* invalid argument (e.g. an id whose key exceeds the universe) */
#define CR_ERR_ALLOC 3        /* device or pinned host allocation failed */
#define CR_ERR_UNSUPPORTED 4  /* request outside what this build implements */
#define CR_ERR_RANGE 5        /* an index out of range (the reference throws std::out_of_range) */

/* ContainerType (include/cu_roaring/types.cuh:7-11). */
#define CR_ARRAY 0
#define CR_BITMAP 1
#define CR_RUN 2
/* SetOp (include/cu_roaring/detail/set_ops.cuh:7-12). */
#define CR_AND 0
#define CR_OR 1
#define CR_ANDNOT 2
#define CR_XOR 3
/* PROMOTE_* (include/cu_roaring/detail/promote.cuh:38-40). */
#define CR_PROMOTE_KEEP_DEFAULT 4096u
#define CR_PROMOTE_ALL 0u
#define CR_PROMOTE_AUTO 0xFFFFFFFFu
/* CRoaring container type codes accepted by cr_upload_containers (src/upload.cpp:21-23). */
#define CR_TC_BITSET 1
#define CR_TC_ARRAY 2
#define CR_TC_RUN 3
/* cr_contains_batch modes. */
/* Modes 0 and 1 answer as GpuRoaringView::contains does, in batched kernels:
 * on an all-bitmap view a copy of its two-load fast path (mode 1 reads a
 * key_index entry once when the whole wave shares a key, as
 * wavefront_contains does); on other layouts mode 0 calls the header function
 * per query and mode 1 runs its lookup rules with each lane's queries searched
 * in lockstep, for wave-coherent (clustered) batches. */
#define CR_QUERY_CONTAINS 0   /* GpuRoaringView::contains per lane */
#define CR_QUERY_WAVEFRONT 1  /* wavefront_contains (== warp_contains) */
/* Modes 2 and 3 always run the header functions wavefront_contains() and
 * GpuRoaringView::contains() one query at a time, on every layout. */
#define CR_QUERY_WAVEFRONT_API 2
#define CR_QUERY_CONTAINS_API 3
/* Mode 4 gives the same answers by partitioning: the queries are sorted by
 * 16-key bucket on the device, each bucket's containers are loaded once into
 * LDS and its queries answered there, and the answers are written back in
 * input order.  Fastest for many uniform queries over a large bitmap (one
 * random memory request per query otherwise; sorted or clustered batches
 * are faster in modes 0/1); it allocates scratch of about 4.8 bytes per query
 * from the library's pool, stream-ordered. */
#define CR_QUERY_PARTITIONED 4

/*
 * Byte-identical to cu_roaring::GpuRoaring (include/cu_roaring/types.cuh:15-54):
 * same field order and types, 120 bytes on LP64.
 */
typedef struct cr_gpu_roaring {
    uint16_t* keys;
    uint8_t* types;
    uint32_t* offsets;
    uint16_t* cardinalities;
    uint32_t n_containers;
    uint32_t universe_size;
    uint64_t total_cardinality;
    uint64_t* bitmap_data;
    uint32_t n_bitmap_containers;
    uint16_t* array_data;
    uint32_t n_array_containers;
    uint32_t array_pool_bytes;
    uint16_t* run_data;
    uint32_t n_run_containers;
    uint32_t run_pool_bytes;
    uint16_t* key_index;
    uint32_t max_key;
    bool negated;
    void* _alloc_base;
} cr_gpu_roaring;

/* Byte-identical to cu_roaring::GpuRoaringView (include/cu_roaring/device/roaring_view.cuh:14-37). */
typedef struct cr_gpu_roaring_view {
    const uint16_t* keys;
    const uint8_t* types;
    const uint32_t* offsets;
    const uint16_t* cardinalities;
    uint32_t n_containers;
    const uint64_t* bitmap_data;
    const uint16_t* array_data;
    const uint16_t* run_data;
    const uint16_t* key_index;
    uint32_t max_key;
    bool all_bitmap;
    bool negated;
} cr_gpu_roaring_view;

/* GpuRoaringMeta (include/cu_roaring/types.cuh:56-63). */
typedef struct cr_meta {
    uint32_t n_containers;
    uint32_t n_bitmap_containers;
    uint32_t n_array_containers;
    uint32_t n_run_containers;
    uint32_t universe_size;
    size_t total_bytes;
} cr_meta;

/*
 * One host container as upload() reads it from a CRoaring roaring_bitmap_t
 * (src/upload.cpp:31-71, 155-225): typecode CR_TC_*, `cardinality` is the
 * element count for bitset/array containers and n_runs for run containers,
 * `data` points to 1024 u64 words, `cardinality` u16 values, or n_runs
 * (start, length) u16 pairs.  Containers are sorted by key.
 */
typedef struct cr_host_container {
    uint16_t key;
    uint8_t typecode;
    int32_t cardinality;
    const void* data;
} cr_host_container;

/*
 * Byte-identical to cu_roaring::v2::GpuRoaringBatch
 * (v2/include/cu_roaring_v2/types.cuh:37-86): N bitmaps in one device block,
 * CSR-style.  container_starts / key_index_starts (n_bitmaps + 1 entries)
 * slice the concatenated per-container metadata and key indices; a key index
 * entry is the LOCAL container index within its bitmap (0xFFFF = absent);
 * offsets are byte offsets into the per-type pools, which the batch shares.
 * The host_* arrays mirror per-bitmap scalars in host memory.  160 bytes on LP64.
 */
typedef struct cr_roaring_batch {
    uint32_t n_bitmaps;
    uint32_t total_containers;
    uint32_t n_bitmap_containers_total;
    uint32_t array_pool_bytes;
    uint32_t run_pool_bytes;
    uint32_t* container_starts;
    uint32_t* key_index_starts;
    uint16_t* keys;
    uint8_t* types;
    uint32_t* offsets;
    uint16_t* cardinalities;
    uint16_t* key_indices;
    uint64_t* bitmap_data;
    uint16_t* array_data;
    uint16_t* run_data;
    const uint64_t* host_total_cardinalities;
    const uint32_t* host_universe_sizes;
    const uint32_t* host_container_starts;
    const uint32_t* host_key_index_starts;
    const uint32_t* host_n_bitmap_containers;
    void* _alloc_base;
    void* _host_meta_base;
} cr_roaring_batch;

/* Byte-identical to cu_roaring::v2::GpuRoaringView (v2/include/cu_roaring_v2/types.cuh:95-107):
 * one bitmap of a batch, its metadata pointers already offset to its slice. */
typedef struct cr_batch_view {
    uint32_t n_containers;
    uint32_t max_key;
    uint16_t* keys;
    uint8_t* types;
    uint32_t* offsets;
    uint16_t* cardinalities;
    uint16_t* key_index;
    uint64_t* bitmap_data;
    uint16_t* array_data;
    uint16_t* run_data;
} cr_batch_view;

typedef void* cr_stream_t;

const char* cr_last_error(void);

/* upload_from_ids (include/cu_roaring/detail/upload_ids.cuh:19-23; src/upload_ids.cu:567-591).
 * `ids` are host ids; they are copied to the device and processed there. */
int cr_upload_from_ids(const uint32_t* ids, uint32_t n_ids, uint32_t universe_size, cr_stream_t stream,
                       uint32_t bitmap_threshold, cr_gpu_roaring* out);
/* Same semantics with device-resident ids (no reference counterpart; the
 * reference always copies host ids, src/upload_ids.cu:310-313). */
int cr_upload_from_device_ids(const uint32_t* d_ids, uint32_t n_ids, uint32_t universe_size, cr_stream_t stream,
                              uint32_t bitmap_threshold, cr_gpu_roaring* out);
/* upload_from_bitset (upload_ids.cuh:48-51; src/upload_ids.cu:872-893). */
int cr_upload_from_bitset(const uint32_t* host_words, uint32_t n_words, uint32_t universe_size, cr_stream_t stream,
                          cr_gpu_roaring* out);
/* upload_from_device_bitset (upload_ids.cuh:53-56; src/upload_ids.cu:806-867). */
int cr_upload_from_device_bitset(const uint32_t* d_words, uint32_t n_words, uint32_t universe_size,
                                 cr_stream_t stream, cr_gpu_roaring* out);
/* upload_impl, the packed single-allocation upload of a host Roaring
 * (include/cu_roaring/detail/upload.cuh:19-32; src/upload.cpp:89-287).
 * `universe_size` 0 means "infer from the last key" (the overload without U).
 * The complement of upload(bm, U) is applied by the caller, which then passes
 * complemented=true and the logical cardinality (src/upload.cpp:296-316). */
int cr_upload_containers(const cr_host_container* containers, uint32_t n, uint32_t universe_size, bool complemented,
                         uint64_t logical_cardinality, cr_stream_t stream, uint32_t bitmap_threshold,
                         cr_gpu_roaring* out);
/* get_meta (upload.cuh:41; src/upload.cpp:31-71), over the same container list. */
int cr_get_meta(const cr_host_container* containers, uint32_t n, cr_meta* out);
/* set_operation (include/cu_roaring/detail/set_ops.cuh:16-19; src/set_ops.cu:567-1207). */
int cr_set_operation(const cr_gpu_roaring* a, const cr_gpu_roaring* b, uint32_t op, cr_stream_t stream,
                     cr_gpu_roaring* out);
/* multi_and (set_ops.cuh:22-24; src/set_ops.cu:1715-1745). */
int cr_multi_and(const cr_gpu_roaring* bitmaps, uint32_t count, cr_stream_t stream, cr_gpu_roaring* out);
/* gpu_roaring_free / gpu_roaring_free_async (upload.cuh:34,39; src/upload.cpp:318-350).
 * Both reset *bm to the empty struct. */
int cr_free(cr_gpu_roaring* bm);
int cr_free_async(cr_gpu_roaring* bm, cr_stream_t stream);
/* resolve_auto_threshold (include/cu_roaring/detail/promote.cuh:75; src/promote.cu:334-367). */
int cr_resolve_auto_threshold(uint32_t universe_size, int device_id, uint32_t* out_threshold);
/* make_view (include/cu_roaring/device/make_view.cuh:9-27). */
int cr_make_view(const cr_gpu_roaring* bm, cr_gpu_roaring_view* out);
/* Batched point queries: out[i] = view.contains(ids[i]) (mode CR_QUERY_CONTAINS)
 * or wavefront_contains(view, ids[i]) (CR_QUERY_WAVEFRONT), as uint32 0/1.
 * The reference exposes contains()/warp_contains() only as device functions
 * (roaring_view.cuh:39, roaring_warp_query.cuh:16); this is the launcher its
 * benches and tests write around them (bench/bench_point_query.cu:123-144). */
int cr_contains_batch(const cr_gpu_roaring_view* view, const uint32_t* d_ids, uint64_t n, uint32_t* d_out,
                      uint32_t mode, cr_stream_t stream);
/* Filtered brute-force top-k (no reference implementation; the reference
 * motivates a fused filtered search in README.md:265).  base: n_base x dim
 * fp32 row-major (device), queries: n_q x dim fp32 (device), filter: a
 * GpuRoaring over [0, n_base) (NULL = no filter).  Writes, per query, the k
 * smallest squared L2 distances ascending (ties: smaller id first) and their
 * ids; slots beyond the number of passing vectors hold +inf and -1.  A
 * filter's total_cardinality, when non-zero, tells the call which path to
 * launch (an understated one costs time, never the answer). */
int cr_topk_filtered(const float* d_base, uint64_t n_base, const float* d_queries, uint32_t n_q, uint32_t dim,
                     const cr_gpu_roaring* filter, uint32_t k, float* d_out_dist, int64_t* d_out_ids,
                     cr_stream_t stream);
/* Tuning of cr_topk_filtered (no counterpart in the reference).  With at most
 * `rows` passing vectors (capped at 262144, the default, and at 1 GiB of
 * estimates: n_q x rows x 4 bytes) every distance estimate is kept and one
 * workgroup per query selects its k from them, in place of the per-chunk
 * candidate lists; 0 turns that path off.  Both paths give the same answer.
 * Process-wide; returns the previous limit. */
uint32_t cr_topk_set_small_limit(uint32_t rows);

/* ---- conversions --------------------------------------------------------
 * These calls are stream-ordered and do NOT synchronise `stream` (the
 * reference's contract for them, decompress.cuh / to_csr.cuh / promote.cuh:45-47).
 * Buffers returned by the *_alloc variants come from hipMalloc; free them
 * with cr_device_free (hipFree). */
/* decompress_to_bitset into a pre-allocated buffer
 * (include/cu_roaring/detail/decompress.cuh:13-16; src/decompress.cu:104-151):
 * d_out[0, n_words) receives the flat bitset, complemented within U when the
 * bitmap is negated.  Writes stay below n_words (the reference's complement
 * pass writes U/32 words whatever n_words is). */
int cr_decompress_to_bitset(const cr_gpu_roaring* bm, uint32_t* d_out, uint32_t n_words, cr_stream_t stream);
/* decompress_to_bitset, allocating (decompress.cuh:10-11; src/decompress.cu:153-162):
 * *n_words = ceil(U / 32); U == 0 gives *d_out = NULL. */
int cr_decompress_to_bitset_alloc(const cr_gpu_roaring* bm, cr_stream_t stream, uint32_t** d_out, uint32_t* n_words);
/* enumerate_ids into a pre-allocated buffer
 * (include/cu_roaring/detail/to_csr.cuh:35; src/to_csr.cu:161-209): the stored
 * ids in ascending order as int64 (negation is ignored, as in the reference);
 * nothing is written when n_containers or total_cardinality is 0.  At most
 * `out_capacity` ids are written (UINT64_MAX: no bound, the reference's
 * behaviour). */
int cr_enumerate_ids(const cr_gpu_roaring* bm, int64_t* d_out, uint64_t out_capacity, cr_stream_t stream);
/* enumerate_ids, allocating (to_csr.cuh:46; src/to_csr.cu:211-220).  The
 * buffer holds total_cardinality ids, or U - total_cardinality for a negated
 * bitmap (whose stored ids the call writes; the reference's buffer would be
 * too small there); *n_out (may be NULL) receives that count.
 * total_cardinality == 0 gives *d_out = NULL. */
int cr_enumerate_ids_alloc(const cr_gpu_roaring* bm, cr_stream_t stream, int64_t** d_out, uint64_t* n_out);
/* The logical cardinality, counted on the device from the containers' bits
 * (popcount for bitmaps, cards for arrays, sum of lengths for runs); a negated
 * bitmap counts its complement within [0, U).  No counterpart in the
 * reference, which has no accessor: set_operation leaves total_cardinality 0
 * (src/set_ops.cu:1162-1175) and a stored card of 0 may mean 65536.
 * Synchronises the stream. */
int cr_cardinality(const cr_gpu_roaring* bm, cr_stream_t stream, uint64_t* out);
/* enumerate_ids without any allocation.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops).  Same output as cr_enumerate_ids.  Its
 * per-container scratch is a fixed 1 MiB device array per device (2 x 65536
 * u64, held until the process ends); bitmaps of more than 65536 containers are
 * rejected with CR_ERR_INVALID.  Every call on a device shares that array, so
 * calls that overlap on one device (other streams or threads) race; calls on
 * one stream are ordered.  The first call on a device looks the array up
 * (with that device current). */
int cr_enumerate_ids_noalloc(const cr_gpu_roaring* bm, int64_t* d_out, uint64_t out_capacity, cr_stream_t stream);
/* promote_to_bitmap (include/cu_roaring/detail/promote.cuh:48; src/promote.cu:233-323):
 * a new all-bitmap GpuRoaring; cardinalities are copied verbatim (a run
 * container's entry keeps its run count), key_index/max_key come from U. */
int cr_promote_to_bitmap(const cr_gpu_roaring* bm, cr_stream_t stream, cr_gpu_roaring* out);
/* promote_auto (promote.cuh:63-64; src/promote.cu:369-385): promote_to_bitmap
 * when resolve_auto_threshold gives PROMOTE_ALL and an array or run container
 * exists, else a deep copy.  device_id -1 = current device. */
int cr_promote_auto(const cr_gpu_roaring* bm, cr_stream_t stream, int device_id, cr_gpu_roaring* out);
/* gpu_roaring_deep_copy (promote.cuh:83; src/promote.cu:178-231). */
int cr_deep_copy(const cr_gpu_roaring* bm, cr_stream_t stream, cr_gpu_roaring* out);

/* ---- Roaring portable format ----------------------------------------------
 * The serialization format of CRoaring's roaring_bitmap_portable_serialize /
 * _deserialize (RoaringFormatSpec).  The reference has no serializer; its
 * from-disk bench loads CRoaring files and upload()s them
 * (bench/CMakeLists.txt:89-93).  These calls synchronise `stream`. */
/* Bytes cr_portable_serialize writes for `bm`. */
int cr_portable_size_in_bytes(const cr_gpu_roaring* bm, cr_stream_t stream, size_t* out_bytes);
/* Serializes the logical set of `bm` (a negated bitmap is complemented within
 * [0, U)) into host memory, each container encoded as CRoaring's run_optimize
 * would leave it (array up to 4096 values, else bitset, run when smaller);
 * empty containers are skipped.  *written receives the size; a buffer smaller
 * than that gives CR_ERR_INVALID. */
int cr_portable_serialize(const cr_gpu_roaring* bm, cr_stream_t stream, void* host_buf, size_t capacity,
                          size_t* written);
/* upload() of a portable-format bitmap held in host memory: the same result as
 * deserializing it with CRoaring and calling upload(bm) (universe_size 0) or
 * upload(bm, universe_size) (include/cu_roaring/detail/upload.cuh:19-32).
 * A malformed buffer (truncated, bad cookie, keys out of order, a run past
 * 0xFFFF) gives CR_ERR_INVALID. */
int cr_portable_deserialize(const void* buf, size_t len, uint32_t universe_size, cr_stream_t stream,
                            uint32_t bitmap_threshold, cr_gpu_roaring* out);

/* ---- the v2 batch API (v2/include/cu_roaring_v2/api.hpp) ------------------
 * Container types are kept as given; only cr_promote_batch changes them. */
/* upload_batch (api.hpp:22-24; v2/src/upload.cpp:319-360): bitmap b is the
 * container list bitmaps[b][0, n_containers[b]) (keys strictly increasing, as
 * in a roaring_bitmap_t).  One device block, one host-to-device copy; synchronises
 * `stream`.  n_bitmaps 0 gives the empty batch. */
int cr_upload_batch(const cr_host_container* const* bitmaps, const uint32_t* n_containers, uint32_t n_bitmaps,
                    cr_stream_t stream, cr_roaring_batch* out);
/* free_batch (api.hpp:28; v2/src/upload.cpp:362-372): synchronises the device,
 * releases both blocks and zeroes *batch. */
int cr_free_batch(cr_roaring_batch* batch);
/* promote_batch (api.hpp:35-36; v2/src/promote.cu:214-304): a new all-bitmap
 * batch; cardinalities recomputed by popcount (65536 stored as 0).
 * Stream-ordered, no synchronisation. */
int cr_promote_batch(const cr_roaring_batch* batch, cr_stream_t stream, cr_roaring_batch* out);
/* make_view (api.hpp:42; v2/src/upload.cpp:374-415).  CR_ERR_RANGE when b >= n_bitmaps. */
int cr_batch_make_view(const cr_roaring_batch* batch, uint32_t b, cr_batch_view* out);
/* multi_and (api.hpp:52-55; v2/src/multi_and.cu:276-470): AND of the bitmaps
 * host_indices[0, n_inputs) (every one all-bitmap, else CR_ERR_INVALID; an
 * index out of range gives CR_ERR_RANGE) into a new 1-bitmap batch.
 * Synchronises `stream` once (the result's counts). */
int cr_batch_multi_and(const cr_roaring_batch* batch, const uint32_t* host_indices, uint32_t n_inputs,
                       cr_stream_t stream, cr_roaring_batch* out);
/* decompress_batch (api.hpp:62-65; v2/src/decompress.cu:151-178): bitmap b's
 * containers into d_bitsets[b * words_each, (b + 1) * words_each): a bitmap
 * container's window is stored, an array / run window OR-ed into the buffer
 * (callers zero it first).  CR_ERR_INVALID when words_each < ceil(max universe / 64). */
int cr_batch_decompress(const cr_roaring_batch* batch, uint64_t* d_bitsets, uint64_t words_each,
                        cr_stream_t stream);
/* Batched contains(batch, b, id) (v2/include/cu_roaring_v2/query.cuh:97-112):
 * d_out[i] = 1 iff bitmap (d_bitmap_idx ? d_bitmap_idx[i] : b) holds d_ids[i].
 * The reference's v2 tests write this launcher around the device function
 * (v2/test/test_basic.cu:47-55). */
int cr_batch_contains(const cr_roaring_batch* batch, const uint32_t* d_bitmap_idx, uint32_t b,
                      const uint32_t* d_ids, uint64_t n, uint8_t* d_out, cr_stream_t stream);
/* Batched contains(view, id) (query.cuh:75-92; v2/test/test_basic.cu:38-45). */
int cr_batch_view_contains(const cr_batch_view* view, const uint32_t* d_ids, uint64_t n, uint8_t* d_out,
                           cr_stream_t stream);

/* ---- utilities (no reference counterpart) -------------------------------- */
/* L2 size the AUTO rule uses for `device_id` (hipDeviceAttributeL2CacheSize). */
int cr_device_l2_bytes(int device_id, uint64_t* out_bytes);
/* Plain device memory helpers for bindings that have no HIP runtime of their own. */
int cr_device_malloc(void** ptr, size_t bytes);
int cr_device_free(void* ptr);
int cr_memcpy_h2d(void* dst, const void* src, size_t bytes);
int cr_memcpy_d2h(void* dst, const void* src, size_t bytes);
int cr_stream_synchronize(cr_stream_t stream);
/* The library allocates results and scratch from its own per-device HIP memory
 * pool, which keeps freed memory cached (release threshold: never) so repeated
 * calls do not remap device memory; blocks it frees on a stream are also kept
 * and reused by later calls on that stream without a runtime call (so a stream
 * must not be destroyed while library work on it is in flight).  Release the
 * cached blocks of `device_id` (-1 = current device) and trim its pool down to
 * `keep_bytes`; synchronises the device. */
int cr_mempool_trim(int device_id, size_t keep_bytes);
/* Per-kernel HIP-event timing: enable (on >= 1) / disable (0) and clear the
 * records; with on = p > 1 only every p-th launch of each kernel is timed.
 * The report is one "kernel_name timed_launches total_ms median_ms" line per
 * kernel (host phases are named "host:<phase>"). */
int cr_timing_enable(int on);
int cr_timing_report(char* buf, size_t cap);
/* Fault injection for tests of the error contract (no counterpart in the
 * reference, whose failures come only from the CUDA runtime): after `skip`
 * more successful device allocations, the next `count` fail as an
 * out-of-memory would, with CR_ERR_ALLOC (count = 0 turns it off).  Process-
 * wide; calls made meanwhile on other threads see it too. */
int cr_debug_fail_device_allocs(uint32_t skip, uint32_t count);

#ifdef __cplusplus
}
#endif
#endif /* CU_ROARING_ABI_H */
