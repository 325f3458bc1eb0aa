/*
 * ltx_loader.h — the block-streaming loader's host side: blob mmap + manifest
 * + layout check, and the 2-slot pinned host ring with a reader thread.
 * Replaces ltx/loader.zig (Blob at :45-92, Ring at :176-321) over the same
 * on-disk format (tools/pack_block.py: blob.bin + blob_manifest.json).
 *
 * Status convention as ltx_block.h: non-zero = success. Error names follow
 * the reference's error set and appear in the error text:
 *   BlobSizeMismatch, Misaligned, LayoutGap, TrailingBytes, MissingEntry,
 *   BlobDigestMismatch, ScheduleOutOfRange, SlotTooSmall, RingShutdown,
 * plus FormatVersion: packer_version must be 1 (the reference format: F32
 * scales, int8 q/k/v and ff only) or 2 (adds F16 scales and int8
 * out-projections), and a version-1 manifest may not use version-2 entries.
 */
#ifndef LTX_LOADER_H
#define LTX_LOADER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ltx_blob ltx_blob;
typedef struct ltx_ring ltx_ring;

/* Blob.open (ltx/loader.zig:50-69): parse DIR/blob_manifest.json, check the
 * size of DIR/blob.bin against total_bytes, mmap it read-only. */
int ltx_blob_open(const char* dir, ltx_blob** out);
void ltx_blob_close(ltx_blob* b);
/* Blob.checkLayout (ltx/loader.zig:73-82). */
int ltx_blob_check_layout(const ltx_blob* b);
/* sha256 of the whole blob against the manifest's blob_sha256. */
int ltx_blob_verify(const ltx_blob* b);
const void* ltx_blob_data(const ltx_blob* b, uint64_t* bytes);
const char* ltx_blob_manifest_text(const ltx_blob* b);
int64_t ltx_blob_block_index(const ltx_blob* b);
/* findEntry by normalised name (ltx/loader.zig:100-129). dtype_out may be NULL. */
int ltx_blob_find(const ltx_blob* b, const char* normalized_name, uint64_t* offset, uint64_t* nbytes, char* dtype_out,
                  int dtype_cap);

/* Ring (ltx/loader.zig:185-321). `schedule` holds indices into `blobs`, one
 * per scheduled block execution. Slots are hipHostMalloc'd pinned memory when
 * `pinned` (requires a GPU runtime), page-aligned host memory otherwise. */
int ltx_ring_create(ltx_blob* const* blobs, int nblobs, const int* schedule, int nsched, int verify_first_touch,
                    uint64_t slot_bytes, int pinned, ltx_ring** out);
/* Ring.staticCheck (ltx/loader.zig:225-235). */
int ltx_ring_static_check(const ltx_ring* r);
/* Spawn the reader thread (Ring.readerMain, ltx/loader.zig:240-287). */
int ltx_ring_start(ltx_ring* r);
/* Ring.acquire (ltx/loader.zig:290-304): block until the slot staging
 * schedule position `pos` is ready; returns its memory. */
int ltx_ring_acquire(ltx_ring* r, int pos, const void** mem, uint64_t* bytes);
/* Ring.release (ltx/loader.zig:315-320) of the slot holding `pos`. */
int ltx_ring_release(ltx_ring* r, int pos);
/* Ring.abort (ltx/loader.zig:306-313): idempotent; retires the reader. */
void ltx_ring_abort(ltx_ring* r);
int ltx_ring_stats(const ltx_ring* r, uint64_t* reader_parks, uint64_t* consumer_parks, uint64_t* copy_ns,
                   uint64_t* verify_ns);
/* Test hook: the reader sleeps `us` microseconds before staging each blob
 * (forces the slow-reader schedule of ltx/ring_dryrun.zig:52-74). */
int ltx_ring_set_reader_delay_us(ltx_ring* r, uint32_t us);
/* abort + join + free. */
void ltx_ring_destroy(ltx_ring* r);

/* Last loader error text of the calling thread. */
const char* ltx_loader_last_error(void);

/* SHA-256 hex digest (65 bytes with the NUL). */
int ltx_sha256_hex(const void* data, uint64_t n, char* out65);

#ifdef __cplusplus
}
#endif
#endif
