/*
 * mnn_debug.h — diagnostic entry points of libmnn.so, kept out of the product header mnn.h.
 * They have no counterpart in the reference; the library's tests use them to check the
 * hardware assumptions its kernels are written against.
 */
#ifndef MNN_DEBUG_H
#define MNN_DEBUG_H

#include "mnn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Runs one MFMA instruction on one wave with a zero accumulator and returns its raw lane
 * registers, to check the operand/result lane layouts the kernels assume.
 * variant 0: f32 32x32x2 (a, b: 64 floats, one per lane; d: 64 x 16)
 * variant 1: f32 16x16x4 (a, b: 64 floats; d: 64 x 4)
 * variant 2: bf16 32x32x16 (a, b: 64 x 8 floats, rounded to bf16; d: 64 x 16)
 * variant 3: bf16 16x16x32 (a, b: 64 x 8 floats, rounded to bf16; d: 64 x 4)
 * Layout of every array: [lane][register]. */
mnn_status mnn_debug_mfma_probe(mnn_device dev, int variant, const float* a, const float* b,
                                float* d);

/* The plan the encoder's implicit-GEMM conv launcher picks for a level (input channels, output
 * channels, output length, batch; gn_finish: the plan of the GroupNorm split-K finish, which
 * always splits K): K split count and output tile. bench.py uses it to account the split-K
 * finish's bytes. */
mnn_status mnn_debug_enc_conv_plan(int in_channels, int out_channels, int64_t out_length,
                                   int batch, int gn_finish, int* splits, int* tile_m,
                                   int* tile_n);

/* Launch log, a profiling aid: while enabled, every kernel launch of the device appends a line
 * "name grid.x grid.y grid.z block.x" (name as in mnn_device_kernel_timing). Enabling clears the
 * log. mnn_debug_launch_log copies it, NUL-terminated, into buf (cap bytes) and sets *needed to
 * the size required; MNN_ERR_BUFFER_SIZE_MISMATCH when cap is too small. A `rocprofv3 --pmc` run
 * of a known sequence of launches is attributed to the library's kernel names this way. */
mnn_status mnn_debug_set_launch_log(mnn_device dev, int enable);
mnn_status mnn_debug_launch_log(mnn_device dev, char* buf, size_t cap, size_t* needed);

/* Bound of the grid-wide wait in one-launch kernels (the Conv1D -> GroupNorm(1) chain of a
 * Sequential): the number of times a workgroup polls for the other workgroups' statistics before
 * it computes them itself. The result is the same either way; 0 makes every workgroup that does
 * not find every partial on its first look take the self-computing path, which the tests use to
 * check it. *previous (may be null) receives the old bound; the default is 65536. */
mnn_status mnn_debug_set_grid_spin_limit(mnn_device dev, int polls, int* previous);

/* Every entry of the device's kernel timing (mnn_device_set_kernel_timing), one line each:
 * "name launches total_ms", names exact (mnn_device_kernel_timing matches substrings). Copied
 * NUL-terminated into buf (cap bytes); *needed = the size required; buf NULL only sizes it,
 * MNN_ERR_BUFFER_SIZE_MISMATCH when cap is too small. */
mnn_status mnn_debug_kernel_timing_table(mnn_device dev, char* buf, size_t cap, size_t* needed);

/* Timing marks: mnn_debug_stream_mark records timing event `index` (0..65535; events are made on
 * first use and kept until the stream is destroyed) on the stream; mnn_debug_stream_mark_elapsed
 * waits for mark `to` and gives the milliseconds between marks `from` and `to`. bench.py brackets
 * each timed call with two marks, so per-call GPU times need no host synchronisation between the
 * calls. */
mnn_status mnn_debug_stream_mark(mnn_stream s, int index);
mnn_status mnn_debug_stream_mark_elapsed(mnn_stream s, int from, int to, float* ms);

/* Measurement floors, enqueued on s: mnn_debug_empty_launch runs an empty kernel (one workgroup
 * of 64 threads); mnn_debug_stream_rw runs one kernel that reads the first read_bytes of src and
 * writes write_bytes to dst (16-byte vectors, every load before the stores; both counts multiples
 * of 16 within their tensors). Timed like a bandwidth-bound kernel of the same traffic, they give
 * the lowest time that traffic takes in one launch on this device. */
mnn_status mnn_debug_empty_launch(mnn_stream s);
mnn_status mnn_debug_stream_rw(mnn_tensor src, int64_t read_bytes, mnn_tensor dst,
                               int64_t write_bytes, mnn_stream s);

/* Number of device allocations (hipMalloc) the library has made in this process: tensors, layer
 * weights and workspaces. The tests read it around a call to check that the call allocated
 * nothing (the allocation-free entry point). */
mnn_status mnn_debug_device_allocations(int64_t* count);

#ifdef __cplusplus
}
#endif
#endif /* MNN_DEBUG_H */
