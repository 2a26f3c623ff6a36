/*
 * Read-only probe of a decode batch's K/V access pattern
 * (libxllm_stream_probe.so, used by bench.py --copy-peak and the default
 * bench line; not part of the operator C-ABI).
 *
 * tile_desc[i] = (byte offset of the tile's first row in both caches) << 5 |
 * valid rows (1..16); tile_bytes = 16 rows x row bytes (1, 2 or 4 KB).
 * waves (a multiple of 4) wavefronts each read an equal, contiguous run of
 * tiles, K then V, with 16-byte nontemporal loads and one tile in flight,
 * and write one word per lane to sink[waves * 64].  Returns 0, or -1 for bad
 * arguments or a failed launch.
 */
#ifndef XLLM_STREAM_PROBE_H
#define XLLM_STREAM_PROBE_H

#ifdef __cplusplus
extern "C" {
#endif

int xllm_stream_probe(const void *key_cache, const void *value_cache, const long long *tile_desc,
                      long long num_tiles, int tile_bytes, int waves, unsigned *sink,
                      void *stream);

#ifdef __cplusplus
}
#endif

#endif
