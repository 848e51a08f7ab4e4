/*
 * metellus_hip.h -- C ABI of the MI355X (gfx950) native shim.
 *
 * Replaces the reference's Objective-C++/nanobind module `metal_backend`
 * (reference: src/metal_backend.mm:253-261), whose seven Python functions are
 * create_buffer, release_buffer, buffer_size, write_buffer, read_buffer,
 * fill_buffer and run_kernel.  Here run_kernel is split into a cached compile
 * (mt_compile) and a launch (mt_launch); the Python wrapper
 * metellus_amd/runtime/hip_backend.py rebuilds the seven functions on top.
 *
 * Conventions
 *   - Every function returns 0 on success and nonzero on failure; the message
 *     of the calling thread's last failure is returned by mt_last_error().
 *   - Buffers are opaque handles >= 1 owned by the shim's registry.
 *   - All device work is ordered on one HIP stream (default priority).
 *     mt_read, mt_sync and timed launches synchronise; everything else is
 *     asynchronous and stream-ordered (frees included).
 *   - Plain pointers and sizes only; no framework types cross this boundary.
 */
#ifndef METELLUS_HIP_H
#define METELLUS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of this thread's last failure ("" if none). */
const char* mt_last_error(void);

/* Select device 0 and create the stream.  Idempotent; called implicitly. */
int mt_init(void);

/* Number of visible HIP devices (0 on a machine without a GPU). */
int mt_device_count(int* count);

/* Target id of device 0 (e.g. "gfx950:sramecc+:xnack-"), compute-unit count
 * and peak clock in kHz. */
int mt_device_info(char* arch, size_t arch_len, int* cu_count, int* clock_khz);

/* No counterpart in the reference.  PCI bus id of device 0
 * ("dddd:bb:dd.f"), its memory clock in kHz and its memory size in bytes
 * (any pointer may be NULL): which GPU a measurement ran on. */
int mt_device_pci(char* bus_id, size_t bus_id_len, int* mem_clock_khz, uint64_t* total_mem);

/* create_buffer (reference: src/metal_backend.mm:94-99): nbytes must be > 0. */
int mt_alloc(size_t nbytes, uint64_t* handle);

/* release_buffer (reference: src/metal_backend.mm:101-103): *existed is 1 if
 * the handle was live, 0 if unknown/already released (not an error).  The
 * device block is kept for reuse by later mt_alloc calls of its size class
 * (blocks >= 2 MiB in 2 MiB steps, smaller ones in 256 B steps; a cached
 * block serves a request up to 1/8 smaller) while the cache holds less than
 * a quarter of the device (at most 64 GiB); returning device memory to the
 * driver halves host<->device copy rates for the next ~50 ms on MI355X.
 * Reuse is stream-ordered, as with hipFreeAsync. */
int mt_free(uint64_t handle, int* existed);

/* No counterpart in the reference (Metal buffers go back to the system when
 * released).  Return every cached device block to the driver; mt_alloc also
 * does this by itself when the device runs out of memory. */
int mt_trim(void);

/* Bytes and blocks in the device block cache (either pointer may be NULL). */
int mt_cache_info(size_t* cached_bytes, size_t* cached_blocks);

/* No counterpart in the reference.  How many device blocks (hipMallocAsync)
 * and page-locked host blocks (hipHostMalloc) the shim has requested from
 * the runtime since the process started, how many buffers its registry holds
 * (the workspace included), and the workspace's size (0: none yet).  Any
 * pointer may be NULL.  Lets a caller check that a call allocated nothing. */
int mt_alloc_stats(uint64_t* device_allocs, uint64_t* host_allocs, uint64_t* live_buffers,
                   size_t* workspace_bytes);

/* buffer_size (reference: src/metal_backend.mm:105-108). */
int mt_size(uint64_t handle, size_t* nbytes);

/* Device address of a buffer (for callers that launch their own work). */
int mt_device_ptr(uint64_t handle, uint64_t* address);

/* write_buffer (reference: src/metal_backend.mm:110-117): copies nbytes from
 * host memory; nbytes must not exceed the buffer size.  Returns after the
 * copy completed.  Copies of >= 4 MiB from pageable memory go through the
 * shim's page-locked staging ring (parallel host copies overlapped with the
 * DMA); page-locked sources are copied directly. */
int mt_write(uint64_t handle, const void* src, size_t nbytes);

/* read_buffer (reference: src/metal_backend.mm:119-126): waits for all
 * queued work, then copies nbytes to host memory (staged like mt_write when
 * the destination is pageable and nbytes >= 4 MiB). */
int mt_read(uint64_t handle, void* dst, size_t nbytes);

/* fill_buffer (reference: src/metal_backend.mm:128-141): byte fill. */
int mt_fill(uint64_t handle, uint8_t value);

/* Page-locked host memory of at least nbytes (no counterpart in the
 * reference, whose buffers are unified memory).  Reads into it run at the
 * link's DMA rate with no staging copy; the Python wrapper backs large
 * downloads with it.  Blocks come from a pool (64 KiB granules) and return
 * to it on mt_host_free; up to 1 GiB of returned blocks stay cached. */
int mt_host_alloc(size_t nbytes, void** ptr);

/* Return a block from mt_host_alloc to the pool (NULL is a no-op). */
int mt_host_free(void* ptr);

/* First half of run_kernel (reference: src/metal_backend.mm:178-207):
 * compile `source` with hiprtc for the device's target, load it and look up
 * `function_name`.  Code objects are cached in memory (and on disk unless
 * MT_KERNEL_CACHE=0) by the exact (source, function, options, target,
 * hiprtc version) key, so repeated dispatches do not recompile; a disk entry
 * stores its key and is used only when that key matches in full.
 * `options` is a space-separated
 * list appended to the defaults (-O3 -std=c++17 -ffp-contract=off, packed
 * fp32 ops disabled). */
int mt_compile(const char* source, const char* function_name, const char* options, uint64_t* kernel);

/* Compile only (no device needed): returns the code-object size for the
 * given target ("gfx950" when NULL).  Used to check generated kernels build
 * on a machine without a GPU. */
int mt_compile_only(const char* source, const char* options, const char* target, size_t* code_size);

/* Second half of run_kernel (reference: src/metal_backend.mm:209-249):
 * launch grid[0..2] workgroups of block[0..2] lanes.  The kernel's
 * parameters are the nbuf buffers in order with the `ndims` uint32 dims
 * (passed by value as a 16-word struct) inserted at position dims_slot.
 * When timed != 0 the launch is bracketed by HIP events on the shim's stream
 * and *ms receives the kernel time after synchronising. */
int mt_launch(uint64_t kernel, const uint64_t* buffers, int nbuf, const uint32_t* dims, int ndims,
              int dims_slot, const uint32_t* grid, const uint32_t* block, int timed, float* ms);

/* Allocation-free variant of mt_launch.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory -- code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * Same parameters and kernel-parameter order as mt_launch, without timing;
 * when scratch_bytes > 0 (the workspace_bytes of a stream-K kernel or of a
 * row-reduction epilogue that combines row blocks across workgroups) the kernel's
 * last parameter is the library's static device scratch instead of the
 * mt_workspace buffer.  The scratch holds at most 64 MiB + 4096 bytes
 * (larger requests fail with an error and launch nothing); its 4096-byte
 * flag head is cleared by a small kernel before each such launch.  The call
 * performs no device or host allocation and requires a prior mt_init (it
 * fails otherwise).  All calls on one device share its scratch, which keeps
 * the last launch's contents: they are ordered by the shim's single stream,
 * but launches that overlap on one GPU by other means (a captured graph
 * replayed on another stream) race.  error == NULL: asynchronous.
 * Otherwise the call waits for the launch and stores the scratch's error
 * word (nonzero: a stream-K wait gave up and the results are invalid). */
int mt_launch_noalloc(uint64_t kernel, const uint64_t* buffers, int nbuf, const uint32_t* dims, int ndims,
                      int dims_slot, const uint32_t* grid, const uint32_t* block, size_t scratch_bytes,
                      uint32_t* error);

/* Timing markers (no counterpart in the reference, whose run_kernel times
 * one dispatch at a time): record marker `slot` (0..15) on the shim's
 * stream, after everything queued so far.  The events skip the system-scope
 * release fence, like timed launches. */
int mt_mark(int slot);

/* Wait for marker `to`, then *ms = GPU time from marker `from` to `to`:
 * several launches queued back to back are timed as one sequence. */
int mt_mark_elapsed(int from, int to, float* ms);

/* Wait for all queued work on the shim's stream. */
int mt_sync(void);

/* Number of kernels compiled by hiprtc in this process (cache misses) and
 * served from a cache (hits); for tests of the cache. */
int mt_cache_stats(uint64_t* compiled, uint64_t* hits);

/* No counterpart in the reference, whose matmul dispatches are one tile per
 * threadgroup (reference: src/compute/matmul/config.py:36-37).  Handle of
 * the shim's device workspace, at least nbytes (>= 4096): a stream-K
 * matmul kernel takes it as its last parameter, after the dims.  Its first
 * 4096 bytes are flag words, zero when created and left zero by every
 * launch that completes; growing it frees the old one in stream order.  The
 * handle belongs to the shim (mt_free refuses it).  Launches that share the
 * workspace are ordered by the shim's single stream. */
int mt_workspace(size_t nbytes, uint64_t* handle);

/* Read (synchronously) and clear the workspace's error word: nonzero when a
 * stream-K workgroup gave up waiting for a partial tile, in which case the
 * results of that launch are invalid and the flag words are reset to 0.
 * *error = 0 when no workspace exists. */
int mt_workspace_check(uint32_t* error);

#ifdef __cplusplus
}
#endif

#endif /* METELLUS_HIP_H */
