/*
 * dizo_amd.h -- C ABI of the MI355X (gfx950) DiZO zeroth-order step kernels.
 *
 * Plain C: no torch or C++ types cross this boundary. Tensors are owned by
 * the caller (PyTorch); the library only stores their device addresses. All
 * functions return DZ_OK (0) or a negative DZ_ERR_* code; dz_last_error()
 * returns the calling thread's last message. Work is enqueued asynchronously
 * on the `stream` argument (a hipStream_t, NULL = legacy default stream);
 * nothing synchronises except dz_table_create/destroy. The caller keeps every
 * registered storage alive and in place while a table refers to it.
 *
 * References below are file:line in luozoupi/DiZO, large_models/trainer.py.
 */
#ifndef DIZO_AMD_H
#define DIZO_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DZ_DTYPE_F32 0
#define DZ_DTYPE_F16 1
#define DZ_DTYPE_BF16 2

#define DZ_OK 0
#define DZ_ERR_INVALID (-1) /* bad argument (null, size, dtype, range)      */
#define DZ_ERR_HIP (-2)     /* a HIP runtime call failed                    */
#define DZ_ERR_DEVICE (-3)  /* current device differs from the table's one   */
#define DZ_ERR_RANGE (-4)   /* pointer range outside its device allocation  */

#define DZ_PROJ_SUMSQ 0         /* partial sums only (norm of theta - theta0)  */
#define DZ_PROJ_APPLY 1         /* theta <- theta0 + (theta - theta0) * alpha  */
#define DZ_PROJ_REVERSE 2       /* theta <- theta0 + (theta - theta0) / alpha  */
#define DZ_PROJ_REVERSE_SUMSQ 3 /* REVERSE, then the norms of the new theta    */
#define DZ_PROJ_APPLY_F32ALPHA 4 /* APPLY with an fp32 alpha, one final rounding */

#define DZ_STREAM_PARAM 0u /* z of parameter perturbation / update */
#define DZ_STREAM_GAMMA 1u /* z of the DiZO gamma perturbation     */
#define DZ_STREAM_INIT 2u  /* synthetic weight initialisation      */

typedef struct dz_table dz_table;

/* Library version (major*10000 + minor*100 + patch). */
int32_t dz_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* dz_last_error(void);

/* ---- host-only helpers (no GPU needed) --------------------------------- */

/* Copies the 32768-entry quantile table Q_T (bit patterns of T) that maps a
 * 15-bit index to |z|: Q_T[i] = RNE_T(Phi^-1(1/2 + (i + 1/2)/65536)).
 * `out` holds n_entries elements of 2 (f16/bf16) or 4 (f32) bytes.
 * Replaces the normal transform inside torch.normal, trainer.py:1441,1607. */
int32_t dz_normal_table(int32_t dtype, void* out, int64_t n_entries);

/* Block of the z generator, Philox4x32-7, for key = seed and the counter words
 * (stream, q mod 2^32, 0, q >> 32), on the host. */
int32_t dz_philox_host(uint64_t seed, uint32_t stream_id, uint64_t q, uint32_t out[4]);

/* ---- parameter tables --------------------------------------------------- */

/* Registers n tensors of one dtype on `device`. ptrs[i] is the device address
 * of tensor i (numels[i] elements, contiguous). With anchor_ptrs == NULL the
 * table is a ZO table (perturb/update); with anchor_ptrs the table is a
 * projection table whose tensor i is group i with anchor theta0_i.
 * z_offsets (may be NULL) gives each tensor's global z index (a multiple of
 * 8); NULL lays the tensors end to end from 0, each rounded up to 8 elements.
 * Each address range is checked against its device allocation. The table
 * holds device memory until dz_table_destroy: 32-byte tile descriptors (one
 * per 32,768 elements of a 16-bit type or 8,192 fp32 elements; a bf16 ZO
 * table also one per 24,576 elements for its restore + update + next
 * perturbation launches; a projection table one per chunk and an fp64
 * partial sum per chunk) and its work counters.
 * Replaces the trainable-set walk of trainer.py:1147-1160 (ZO table) and the
 * exclude_list walk of trainer.py:405-451, 581-584 (projection table). */
int32_t dz_table_create(const uint64_t* ptrs, const uint64_t* anchor_ptrs, const int64_t* numels,
                        const uint64_t* z_offsets, int32_t n, int32_t dtype, int32_t device,
                        dz_table** out);
int32_t dz_table_destroy(dz_table* t);

/* 1 if the table was built from exactly these n addresses, else 0 (<0 on error). */
int32_t dz_table_matches(const dz_table* t, const uint64_t* ptrs, int32_t n);

/* Global z offset (element index of the tensor's first element) of tensor idx. */
int32_t dz_table_z_offset(const dz_table* t, int32_t idx, uint64_t* out);

/* Measurement hook; no counterpart in the reference (it serves the bench's
 * per-pass timing). The next call on `t` that launches kernels (dz_perturb,
 * dz_update, dz_restore_update, dz_restore_update_perturb, dz_group_sumsq,
 * dz_project, dz_group_dot) records start_event when its first kernel starts
 * and stop_event when its last kernel ends, through hipExtLaunchKernel, so
 * the pair times the kernels without the host's launch work. Either may be
 * NULL. Both are hipEvent_t handles the caller created (and has recorded at
 * least once). The request is taken by that next call: one with nothing to
 * launch (every tensor empty) records both on its stream at once, one that
 * fails records neither. Do not set it on a stream being captured into a
 * graph. */
int32_t dz_table_time_next(dz_table* t, void* start_event, void* stop_event);

/* Tuning hook (no counterpart in the reference): the fused
 * restore+update+next perturb pass of a table runs its prefetching tile
 * loop (the next tile loaded while the current one computes) only for
 * launches of at least min_tiles tiles; smaller launches run the plain loop.
 * The default, 0, selects it for every launch: measured on the MI355X in the
 * ZO step it is the faster loop at 10 K fp32 tiles (OPT-125m), 77 K fp16
 * tiles (OPT-2.7B) and 384 K (OPT-13B). Tests set a large value to run the plain loop. The values the
 * passes compute do not depend on it. */
int32_t dz_table_set_prefetch_min_tiles(dz_table* t, uint32_t min_tiles);

/* ---- ZO step (trainer.py:1429-1444, 1570-1617) -------------------------- */
/* Launches on one table share its work counters: order them on one stream
 * (never run two launches of the same table concurrently).
 * Optional device pointers (NULL = use the by-value argument):
 *   d_seed: uint64 seed;  d_grad: projected_grad as one element of the table
 *   dtype;  d_lr: fp32 learning rate. They let a captured graph replay with
 *   new values. */

/* theta <- R(theta + R(R(scale*z)*eps)) for every registered tensor.
 * Replaces zo_perturb_parameters(random_seed, scaling_factor), trainer.py:1429-1444. */
int32_t dz_perturb(dz_table* t, uint64_t seed, float scale, float eps, const uint64_t* d_seed,
                   void* stream);

/* theta <- R(theta - R(lr*R(grad*z))).
 * Replaces the parameter loop of zo_update, trainer.py:1603-1608. */
int32_t dz_update(dz_table* t, uint64_t seed, float grad, float lr, const uint64_t* d_seed,
                  const void* d_grad, const float* d_lr, void* stream);

/* The restore of zo_step (scaling_factor = +1, trainer.py:1593) followed by
 * the update of zo_update (trainer.py:1603-1608), in one pass: z is
 * regenerated once and every element is read and written once. */
int32_t dz_restore_update(dz_table* t, uint64_t seed, float eps, float grad, float lr,
                          const uint64_t* d_seed, const void* d_grad, const float* d_lr,
                          void* stream);

/* The fused restore+update of step k (as dz_restore_update, z from `seed`)
 * followed by the first perturbation (+1, same eps) of step k+1 (z from
 * `next_seed`), in one pass: trainer.py:1593 and 1603-1608 of step k, then
 * trainer.py:1580 of the next zo_step. Per element the three operations are
 * applied in that order with the reference's rounding. */
int32_t dz_restore_update_perturb(dz_table* t, uint64_t seed, uint64_t next_seed, float eps, float grad,
                                  float lr, const uint64_t* d_seed, const uint64_t* d_next_seed,
                                  const void* d_grad, const float* d_lr, void* stream);

/* ---- z export / RNG (test and tooling use) ------------------------------ */

/* n normals z(seed, stream_id, offset + i) in `dtype`, written densely to d_out.
 * The materialised z of trainer.py:1441 (random_vector, :1444). */
int32_t dz_normals(uint64_t seed, uint32_t stream_id, uint64_t offset, int64_t n, int32_t dtype,
                   void* d_out, void* stream);

/* The z that dz_perturb/dz_update apply to tensor idx of a ZO table. */
int32_t dz_export_z(const dz_table* t, uint64_t seed, int32_t idx, void* d_out, void* stream);

/* n blocks of the z generator, Philox4x32-7 (4 x uint32 each), for counters q0 .. q0+n-1. */
int32_t dz_philox(uint64_t seed, uint32_t stream_id, uint64_t q0, int64_t n, uint32_t* d_out,
                  void* stream);

/* ---- DiZO projection (trainer.py:405-465, 564-614) ----------------------- */
/* As for the ZO launches, launches on one projection table share its work
 * counters: order them on one stream. */

/* Per group g: d_sumsq[g] = sum fp32(R(theta-theta0))^2 (fp64 accumulation),
 * d_norm_f32[g] = sqrt_f32(fp32(sumsq)), d_norm_T[g] = R_T(norm): the
 * torch.norm(theta - theta0) of trainer.py:455-457 and :583. Any output may be NULL. */
int32_t dz_group_sumsq(dz_table* t, double* d_sumsq, float* d_norm_f32, void* d_norm_T,
                       void* stream);

/* Set-up of the allocation-free entry point on `device`, which must be the
 * current device: loads the library's device code there, resolves the
 * address of its static scratch array and makes one empty kernel launch (the
 * runtime allocates for a library's first launch on a device), then waits
 * for it on the null stream. No counterpart in the reference. For
 * callers that cannot allocate (below): call it once per device before the
 * first dz_group_sumsq_static on that device, outside any graph capture (the
 * HIP runtime loads a library's device code on first use, which allocates).
 * Returns DZ_ERR_DEVICE if `device` is not the current device. */
int32_t dz_init(int32_t device);

/* dz_group_sumsq without a table and without allocating: no counterpart in
 * the reference. For callers that cannot allocate device memory (code under
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). The n
 * groups are theta ptrs[g] with anchors anchor_ptrs[g], numels[g] elements of
 * `dtype` each; the outputs are dz_group_sumsq's, bit for bit. Chunk
 * descriptors, partial sums and work counters live in a static device array
 * of the library (10.5 MB per device, held until the process ends): at most
 * 4096 groups and 262,144 chunks of 32,768 elements of a 16-bit type (8.6 G
 * elements) or of 8,192 fp32 elements (2.1 G); larger inputs return
 * DZ_ERR_INVALID. Every call on one device shares that array,
 * so calls that overlap in time on one device race: order them on one
 * stream. After dz_init(device) a call allocates nothing; without it, the
 * first call on a device does dz_init's work itself. */
int32_t dz_group_sumsq_static(const uint64_t* ptrs, const uint64_t* anchor_ptrs, const int64_t* numels,
                              int32_t n, int32_t dtype, double* d_sumsq, float* d_norm_f32, void* d_norm_T,
                              void* stream);

/* mode DZ_PROJ_APPLY / DZ_PROJ_REVERSE / DZ_PROJ_REVERSE_SUMSQ with one alpha
 * per group (device array of the table dtype). APPLY replaces the copy_ of
 * apply_constraints (trainer.py:428-436); REVERSE replaces reverse_constraints
 * (trainer.py:447-451); REVERSE_SUMSQ also writes the norms of the reversed
 * theta (the next _project_ratio, trainer.py:455-457) to the outputs. */
int32_t dz_project(dz_table* t, const void* d_alpha, int32_t mode, double* d_sumsq,
                   float* d_norm_f32, void* d_norm_T, void* stream);
/* (mode DZ_PROJ_APPLY_F32ALPHA takes one fp32 alpha per group and computes
 * theta <- R_T(fp32(R_T(theta - theta0)) * alpha + theta0): apply_constraints
 * with the fp32 gamma of the first-order path, trainer.py:428-436, 714-741.) */

/* Per group g: d_dot[g] = sum fp32(other_g) * fp32(R_T(theta_g - theta0_g))
 * (fp64 accumulation; d_dot_f32[g] its fp32 rounding), with other_ptrs a host
 * array of n device addresses of tensors shaped like theta_g. The
 * gradient of the first-order gamma objective with respect to alpha
 * (autograd through trainer.py:428-429 in DiZO.forward, trainer.py:714-741). */
int32_t dz_group_dot(dz_table* t, const uint64_t* other_ptrs, double* d_dot, float* d_dot_f32,
                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DIZO_AMD_H */
