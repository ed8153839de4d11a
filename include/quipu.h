/*
 * quipu.h -- C ABI of the MI355X (gfx950) token-loop backend.
 *
 * This library replaces the device side of quipullm's WebGPU engine: the GPU facade of web/js/gpu.js
 * (device, buffers, named pipelines, bind groups, dispatch) and the WGSL kernels it runs.  The JavaScript
 * host (model classes, token loop) binds these entry points through an N-API addon; tests bind them with
 * ctypes.  Every call returns 0 on success, a positive hipError_t value for a HIP failure, or a negative
 * QP_E_* code; qp_last_error() gives the message of the last failure on the calling thread.
 *
 * Buffers are device addresses carried as uint64_t, owned by the caller until qp_free().  One device and
 * one in-order stream per process; calls come from one host thread (the reference engine is single
 * threaded: one job at a time, web/js/engine.js:387-405).  Work is asynchronous except qp_download,
 * qp_sync and qp_event_elapsed.
 */
#ifndef QUIPU_H
#define QUIPU_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QP_E_NOT_INIT (-1)   /* qp_init has not succeeded */
#define QP_E_ARG (-2)        /* bad argument (size, shape, binding count, unknown op) */
#define QP_E_INJECTED (-3)   /* failure forced by QP_FAIL_ALLOC / QP_FAIL_LAUNCH (tests of error paths) */
#define QP_E_CAPTURE (-4)    /* call not allowed while a graph is being captured */

/* ---------------------------------------------------------------- device (GPU.crear, gpu.js:1168-1193) */
/* Opens `device`, creates the stream and loads the kernel code object (QP_KERNELS or quipu_kernels.hsaco
 * next to this library).  Replaces GPU.crear (web/js/gpu.js:1168-1182). */
int qp_init(int device);
/* JSON {"summary","arch","cus","hbm_bytes","max_buffer","bytes_used"} -- gpu.info (gpu.js:1186-1193). */
int qp_info(char* json, size_t cap);
/* Message of the last failure on this thread (empty when none). */
int qp_last_error(char* buf, size_t cap);
/* Device bytes currently allocated through qp_alloc -- gpu.bytesUsados (gpu.js:1194, 1232). */
uint64_t qp_bytes_used(void);
/* 1 after a fatal device error (every later call fails) -- gpu.perdido (gpu.js:1196). */
int qp_lost(void);

/* ---------------------------------------------------------------- buffers (gpu.js:1226-1267) */
/* Device buffer of max(16, roundup(bytes, 4)) bytes, 256-byte aligned -- gpu.buffer (gpu.js:1226-1233). */
int qp_alloc(uint64_t bytes, uint64_t* dev);
/* gpu.liberar (gpu.js:1263-1267). */
int qp_free(uint64_t dev);
/* Host -> device copy, ordered on the stream -- queue.writeBuffer / gpu.subir (gpu.js:1235-1246). */
int qp_upload(uint64_t dst, uint64_t dst_off, const void* src, uint64_t n);
/* Device -> host copy; waits for queued work -- the mapAsync readback (web/js/transformer.js:330-332). */
int qp_download(void* dst, uint64_t src, uint64_t src_off, uint64_t n);
/* Device -> device copy on the stream -- copyBufferToBuffer (web/js/transformer.js:321). */
int qp_copy(uint64_t dst, uint64_t dst_off, uint64_t src, uint64_t src_off, uint64_t n);
/* Waits for all queued work -- queue.onSubmittedWorkDone (web/js/engine.js:284). */
int qp_sync(void);

/* ---------------------------------------------------------------- pipelines and dispatch (gpu.js:1197-1282) */
/* Identifier of a named op (reference kernel names such as "matmul_q4k_1", "rmsnorm", "atencion", plus this
 * backend's fused ops); -1 if unknown -- GPU.pipeline(name) (gpu.js:1197-1212). */
int qp_op_id(const char* name);
/* Runs op `op` with the reference binding list: `uniform` holds binding 0 (the per-op struct P, 16-byte
 * padded as gpu.uniforme builds it, gpu.js:1248-1256), bufs[0] is binding 1 (the Paso step record) and
 * bufs[1..] the storage buffers in binding order (gpu.js:1258-1262).  (gx, gy, gz) is the reference's
 * dispatch size (despachar, gpu.js:1270-1274), from which T-dependent extents are taken; the launch shape
 * itself is the op's own. */
int qp_dispatch(int op, const void* uniform, uint32_t uniform_size, const uint64_t* bufs, uint32_t nbuf,
                uint32_t gx, uint32_t gy, uint32_t gz);

/* qp_dispatch for callers that cannot allocate (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc); no counterpart in the reference.  The same ops as qp_dispatch, and no allocation: the prefill matmul
 * (matmul_<fmt>_4 / _t / _t_swiglu), whose workspace qp_dispatch grows with hipMalloc, takes it from a fixed device
 * array of 32 MiB that each device holds from qp_init until the process ends.  Its split input planes (4 bytes per
 * input value, the tokens rounded up to whole tiles) must fit: up to 512 tokens at K = 14336, 2048 at K = 4096; a
 * call that needs more fails with QP_E_ARG.  Where qp_dispatch's split-K partials would not fit beside them, the
 * K range is split fewer times (the same results up to the order of the partial sums, within the matmul's error
 * bound; bit-identical where nothing is lowered).  Every call on a device shares that array and finds the last
 * call's contents; calls that overlap on one device race. */
int qp_dispatch_noalloc(int op, const void* uniform, uint32_t uniform_size, const uint64_t* bufs, uint32_t nbuf,
                        uint32_t gx, uint32_t gy, uint32_t gz);
/* ---------------------------------------------------------------- raw code objects (no reference counterpart) */
/* hipModuleLoad of a gfx950 code object; hipModuleGetFunction; hipModuleLaunchKernel with one packed
 * argument block.  For host code that brings its own kernels. */
int qp_module_load(const char* path, uint64_t* module);
int qp_kernel(uint64_t module, const char* name, uint64_t* fn);
int qp_launch(uint64_t fn, const uint32_t grid[3], const uint32_t block[3], uint32_t lds, const void* args,
              uint64_t args_size);

/* ---------------------------------------------------------------- graphs and events (no reference counterpart;
 * the reference encodes one command buffer per forward, transformer.js:263-322) */
/* Capture the ops issued between begin and end into a HIP graph; launch replays them. */
int qp_graph_begin(void);
int qp_graph_end(uint64_t* graph);
int qp_graph_launch(uint64_t graph);
int qp_graph_free(uint64_t graph);
int qp_event_create(uint64_t* ev);
int qp_event_record(uint64_t ev);
int qp_event_elapsed(uint64_t ev0, uint64_t ev1, float* ms);
int qp_event_free(uint64_t ev);

#ifdef __cplusplus
}
#endif
#endif
