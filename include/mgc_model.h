/* C ABI of one model compiled by the `hip` backend of ml-graph-compiler.
 *
 * The emitter generates one C++ translation unit per model (host code only: one launcher call
 * into libmgc_hip.so per scheduled node, with every arena and weights offset a constant). Built
 * into lib<name>.so, it exports the symbols below. The first group keeps the names, signatures
 * and meaning of the C backend's exports so that a caller that binds them through ctypes (the
 * reference's CompiledModel) binds a hip model the same way; the second group is what a GPU
 * model needs beyond them.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   mgc_run, mgc_arena_bytes, mgc_weights_bytes     src/ml_graph_compiler/codegen/c.py:1308-1312
 *   mgc_set_num_threads, mgc_get_max_threads,
 *   mgc_has_openmp, mgc_has_neon, mgc_set_blocking  codegen/runtime/mgc_kernels.c:34-70
 *   mgc_profile_size, mgc_profile_data               codegen/c.py:1298-1306 (profile=True only)
 *   binding site                                     codegen/runtime_lib.py:59-68,135-141
 */
#ifndef MGC_MODEL_H
#define MGC_MODEL_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* --- same contract as the C backend ------------------------------------------------------ */

/* Bytes of the planner's arena (memory.py plan, 256-byte aligned offsets) and of the weights
 * blob the emitter wrote next to the library. */
size_t mgc_arena_bytes(void);
size_t mgc_weights_bytes(void);

/* Run the model once. inputs/outputs are HOST pointers in graph input order and named-output
 * order; A and W are the DEVICE arena and weights pointers returned by mgc_hip_init. Returns 0,
 * 1 when a Gather index was out of range, 2 on a HIP runtime error, 3 on bad arguments. */
int mgc_run(const void *const *inputs, void *const *outputs, unsigned char *A,
            const unsigned char *W);

/* Threading and blocking knobs of the CPU backend: accepted and ignored on the GPU
 * (mgc_get_max_threads returns 1, mgc_has_openmp and mgc_has_neon return 0). */
void mgc_set_num_threads(int n);
int mgc_get_max_threads(void);
int mgc_has_openmp(void);
int mgc_has_neon(void);
void mgc_set_blocking(int mc, int kc, int npb);

/* Only in models compiled with profile=True: per-node seconds, accumulated over
 * mgc_hip_profile_run calls (hipEvent pairs around each node's launches). */
int mgc_profile_size(void);
const double *mgc_profile_data(void);

/* --- hip additions ----------------------------------------------------------------------- */

/* Allocate the model's single HBM block, upload weights_host (mgc_weights_bytes bytes) once and
 * return the device arena (*A) and weights (*W) pointers. Calling it again returns the same
 * pointers. */
int mgc_hip_init(const unsigned char *weights_host, unsigned char **A, unsigned char **W);

/* Like mgc_run with DEVICE inputs/outputs (no host copies). */
int mgc_run_device(const void *const *inputs, void *const *outputs, unsigned char *A,
                   const unsigned char *W);

/* Benchmark support: stage host inputs once, enqueue `replays` hipGraph replays, wait. */
int mgc_hip_upload(const void *const *inputs);
int mgc_hip_launch(int replays);
int mgc_hip_sync(void);
int mgc_hip_download(void *const *outputs);
double mgc_hip_time_graph(int replays);

/* profile=True only: eager replays with per-node hipEvent timing; reset the accumulators. */
int mgc_hip_profile_run(int replays);
void mgc_hip_profile_reset(void);

/* Free the model's device memory (the next mgc_hip_init allocates again). */
void mgc_hip_release(void);

#ifdef __cplusplus
}
#endif

#endif /* MGC_MODEL_H */
