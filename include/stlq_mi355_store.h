/*
 * stlq_mi355 — the BaseBasicStore output of the streaming base encode, C ABI.
 *
 * The streaming encode of the reference writes each encoded block to an on-disk store through
 * io::BaseBasicWriter (include/stlq/io/base_store.h:28-100, src/io/base_store.cpp) and, when
 * checkpointing, commits a checkpoint after every block (StreamingBasicCommitHook,
 * include/stlq/quantizer/encode_base_streaming.h:23-28; the pipeline's hook
 * src/pipeline/main_virtual_helpers.cpp:165-297). These entry points write the same files,
 * byte for byte:
 *
 *   meta.json, meta.bin        store parameters (meta.bin: 10 x 32-bit header, then h_vec)
 *   cluster_id.u32             one uint32 per vector, global id order
 *   codes_shard_SSSS.bin       (m-1) uint8 codes per vector, shard_size vectors per shard
 *   coeffs_shard_SSSS.bin      m float coefficients per vector
 *   bucket_BBBB.bin            records of the vectors whose cluster id / bucket_size == BBBB:
 *                              uint32 global id, uint32 cluster id, [raw vector bytes],
 *                              [(m-1) codes, m float coefficients]
 *   checkpoint/base_basic/ckpt.bin   (with checkpointing) magic "BCKT", version 1, nbucket,
 *                              reserved, uint64 next id, nbucket x uint64 committed bucket bytes
 *
 * A block is written into the shard of its first global id (the reference does not split a
 * block at a shard boundary). Host code only; errors follow stlq_mi355.h (status code plus
 * stlq_mi355_last_error()).
 */
#ifndef STLQ_MI355_STORE_H_
#define STLQ_MI355_STORE_H_

#include <stdint.h>

#include "stlq_mi355.h"

#ifdef __cplusplus
extern "C" {
#endif

/* io::BaseBasicStoreConfig (include/stlq/io/base_store.h:12-25). */
typedef struct stlq_mi355_store_config {
    const char* dir;
    int d;
    int m;                     /* layers, the root included: m-1 codes and m coefficients per vector */
    const int* h_vec;          /* m codebook sizes; h_vec[0] (the root) sets the bucket count */
    int h_len;
    int shard_size;            /* default 2,000,000 */
    int bucket_size;           /* cluster ids per bucket file, default 256 */
    int bucket_flush_mb;       /* per-bucket write buffer, default 256 MiB */
    int write_vector_bucket;   /* raw vector bytes in bucket records, default on */
    int write_basic_to_bucket; /* codes + coefficients in bucket records, default on */
    int raw_bytes_per_vec;     /* 0: d (uint8 vectors); d*4 for float vectors */
} stlq_mi355_store_config;

/* Fills the reference's defaults (base_store.h:12-25); dir, d, m and h_vec stay for the caller. */
void stlq_mi355_store_config_init(stlq_mi355_store_config* cfg);

typedef struct stlq_mi355_store stlq_mi355_store;

/* BaseBasicWriter::Open (src/io/base_store.cpp:87-190): creates dir, empties every bucket file
 * of ceil(h_vec[0] / bucket_size) buckets, writes meta.json and meta.bin, truncates
 * cluster_id.u32. */
int stlq_mi355_store_open(const stlq_mi355_store_config* cfg, stlq_mi355_store** out);

/* BaseBasicWriter::OpenResume (src/io/base_store.cpp:192-265): continues a store the caller has
 * truncated to a checkpoint (stlq_mi355_store_truncate_to_checkpoint). start_id is the next global
 * id; bucket_sizes (nbucket entries, nbucket == ceil(h_vec[0] / bucket_size)) are the committed
 * bucket bytes at start_id. Shard and bucket files are appended to. */
int stlq_mi355_store_open_resume(const stlq_mi355_store_config* cfg, uint64_t start_id,
                                 const uint64_t* bucket_sizes, int64_t nbucket, stlq_mi355_store** out);

/* Raw vectors of a block's bucket records. */
#define STLQ_MI355_RAW_NONE 0 /* BaseBasicWriter::AppendBlock(..., x_u8_optional = nullptr, ...) */
#define STLQ_MI355_RAW_U8 1   /* AppendBlockRawU8: raw is uint8, column stride ld_raw >= d */
#define STLQ_MI355_RAW_F32 2  /* AppendBlockRawF32: raw is float, column stride ld_raw >= d */

/* BaseBasicWriter::AppendBlock / AppendBlockRawU8 / AppendBlockRawF32
 * (src/io/base_store.cpp:412-760): appends `count` vectors with global ids start_id.. .
 * cluster_id (count); B_small (b_rows x count, b_rows must be m-1); a (a_rows x count, a_rows
 * must be m). With RAW_U8/RAW_F32 the raw-vector checks come before anything is written; with
 * RAW_NONE and write_vector_bucket set, the block's cluster ids, codes and coefficients are written
 * and then the call fails, as the reference's AppendBlock does. count == 0 writes nothing. */
int stlq_mi355_store_append(stlq_mi355_store* st, uint64_t start_id, int64_t count,
                            const uint32_t* cluster_id, int b_rows, const uint8_t* B_small, int a_rows,
                            const float* a, int raw_kind, const void* raw, int64_t ld_raw);

/* BaseBasicWriter::Flush (src/io/base_store.cpp:290-330): writes out the bucket buffers and
 * flushes every file (no fsync). */
int stlq_mi355_store_flush(stlq_mi355_store* st);

/* BaseBasicWriter::bucket_file_bytes (base_store.h:46): committed on-disk bytes per bucket of
 * the Open/OpenResume layout (buffered records excluded). Writes min(cap, count) entries to out
 * (nullable) and the count to *nbucket (nullable). */
int stlq_mi355_store_bucket_bytes(const stlq_mi355_store* st, uint64_t* out, int64_t cap, int64_t* nbucket);

/* The store's d, m, h_vec[0], write_vector_bucket and raw bytes per bucket record (each nullable). */
int stlq_mi355_store_info(const stlq_mi355_store* st, int* d, int* m, int* h0, int* write_vector_bucket,
                          int* raw_bytes_per_vec);

/* BaseBasicWriter::Close (src/io/base_store.cpp:269-288) and destruction: writes out the buffers,
 * closes the files and frees st (also when Close fails). NULL is a no-op. */
int stlq_mi355_store_close(stlq_mi355_store* st);

/* Checkpoint of a store, src/pipeline/main_virtual_helpers.cpp:100-297.
 * path: <dir>/checkpoint/base_basic/ckpt.bin (BaseBasicCheckpointPath, :122-124). */

/* WriteBaseBasicCheckpointAtomic (:165-206): writes path.tmp, then renames it to path. */
int stlq_mi355_checkpoint_write(const char* path, uint64_t next_id, const uint64_t* bucket_sizes,
                                int64_t nbucket);

/* ReadBaseBasicCheckpoint (:126-163): *next_id, *nbucket and min(cap, nbucket) bucket sizes. */
int stlq_mi355_checkpoint_read(const char* path, uint64_t* next_id, uint64_t* bucket_sizes, int64_t cap,
                               int64_t* nbucket);

/* TruncateBaseBasicToCheckpoint (:208-275): cuts cluster_id.u32, the shard of next_id and every
 * bucket file back to the checkpoint (creating missing files). */
int stlq_mi355_store_truncate_to_checkpoint(const stlq_mi355_store_config* cfg, uint64_t next_id,
                                            const uint64_t* bucket_sizes, int64_t nbucket);

/* EncodeBaseStreaming / EncodeBaseStreamingF32 writing to a store
 * (src/quantizer/encode_base_streaming.cpp:1913-2060, :3060-3212, :3285-3420): the streaming
 * encode of stlq_mi355_encode_stream (chunk == the reference's large.base_block), each chunk
 * appended in order, the raw input tile in its bucket records when the store writes vector
 * buckets (uint8 for input_u8, float otherwise), then, with checkpoint_path non-NULL, the
 * block committed: store flushed and checkpoint written with next id = chunk end
 * (CommitBlock, :2054-2059, and OnCommitBaseBasicCkpt). The store's m must be the encode's m and
 * its h_vec[0] the root codebook size. Coefficients are always produced. With a checkpoint,
 * params->start_id must be a multiple of chunk (:2046-2052). */
int stlq_mi355_encode_stream_store(stlq_mi355_ctx* ctx, int64_t n_total, int64_t chunk,
                                   const stlq_mi355_stream_params* params, stlq_mi355_fill_fn fill,
                                   void* user, stlq_mi355_store* store, const char* checkpoint_path,
                                   stlq_mi355_stream_stats* stats);

#ifdef __cplusplus
}
#endif

#endif /* STLQ_MI355_STORE_H_ */
