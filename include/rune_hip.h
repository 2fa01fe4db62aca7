/*
 * rune_hip.h -- C ABI of the MI355X-native RUNE potential-evaluation path.
 *
 * The reference evaluates energies, forces and virials in PyTorch
 * (rune/mobius/model.py:307-393, rune/nep/model.py:87-155) behind its plugin
 * API (rune/mobius/plugin.py:125-154, rune/nep/plugin.py:57-97).  It has no
 * foreign-function interface of its own; the entry points below are what a
 * binding of that path needs.  Each cites the reference interface it replaces.
 *
 * Conventions
 *   - Plain pointers and sizes only.  "d_" pointers are HIP device memory,
 *     "h_" pointers are host memory.  Streams are hipStream_t passed as void*.
 *   - Every function returns RUNE_OK (0) or an error code; the message of the
 *     last failing call on the calling thread is rune_last_error().
 *   - A handle is used by one host thread / one stream at a time.
 *   - All reductions are deterministic: the same inputs give bitwise identical
 *     outputs on every call (no floating-point atomics anywhere).
 */
#ifndef RUNE_HIP_H
#define RUNE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    RUNE_OK = 0,
    RUNE_ERR_ARGUMENT = 1,   /* bad shape, size, name or configuration        */
    RUNE_ERR_HIP = 2,        /* a HIP runtime call failed                     */
    RUNE_ERR_OVERFLOW = 3,   /* neighbour count exceeds max_neighbors          */
    RUNE_ERR_TYPE = 4,       /* atom type outside [0, n_types)                */
    RUNE_ERR_STATE = 5       /* handle not finalised / inputs inconsistent     */
};

/* Message of the last failing call on this thread ("" if none). */
const char *rune_last_error(void);

/* Version string of the library build. */
const char *rune_version(void);

/* ------------------------------------------------------------------------
 * Neighbour lists.
 *
 * Replaces ase.neighborlist.neighbor_list("ijS", ...) followed by the fp64
 * radial/angular split and padding of
 * rune/mobius/interface/batch.py:42-102 (same in rune/nep/interface/batch.py).
 *
 * Records.  Edges are stored once per centre as "records" e in [0, E):
 *   nbr[e]      neighbour atom (int32, global index)
 *   vec[e]      float4 {x, y, z, |r|}: x,y,z = (fp32(p_j) + fp32(S.cell)) - fp32(p_i)
 *   shift[e]    int32[3] periodic image S (pbc directions only)
 * Records of centre i occupy [ptr[i], ptr[i+1]).  view[4*i + 0..3] =
 * {radial_begin, radial_end, angular_begin, angular_end} are absolute record
 * ranges of the two lists; built lists order each centre's records by
 * (class, j, S0, S1, S2) where class 0 = inside both cutoffs, so the list of
 * the smaller cutoff is a prefix of the segment.
 * ---------------------------------------------------------------------- */
typedef struct rune_nlist rune_nlist;

int rune_nlist_create(rune_nlist **out);
void rune_nlist_destroy(rune_nlist *nl);

/* Build the canonical lists of B structures (atoms of structure b are
 * [h_struct_ptr[b], h_struct_ptr[b+1])).  d_positions: fp64 [N,3] device.
 * h_cells: fp64 [B,3,3] host, rows are lattice vectors; h_pbc: int32 [B,3].
 * A degenerate cell row is allowed only in a non-periodic direction.
 * On success *n_records receives E.  Exceeding max_radial / max_angular
 * returns RUNE_ERR_OVERFLOW with the reference's message. */
int rune_nlist_build(rune_nlist *nl, int64_t n_atoms, const double *d_positions,
                     int32_t n_structures, const int64_t *h_struct_ptr,
                     const double *h_cells, const int32_t *h_pbc,
                     double rc_radial, double rc_angular,
                     int32_t max_radial, int32_t max_angular,
                     void *stream, int64_t *n_records);

/* Verlet-skin reuse of the lists for a moving system (MD loop): same
 * arguments and records as rune_nlist_build, plus `skin` (Angstrom, > 0).
 * The handle keeps the candidates within max(rc) + skin found by its last
 * search and the positions that search saw; a call searches again only when
 * it is the first, when the atom count, structure ranges, cells, pbc,
 * cutoffs, limits or skin changed, or when some atom moved by skin / 2 or
 * more (positions compared as given: an atom wrapped into the cell also
 * triggers a search).  Otherwise the candidates are re-tested at the current
 * positions with the same exact fp64 test, so the records are bitwise those
 * of rune_nlist_build on the same positions either way.  *searched (may be
 * NULL) receives 1 when this call searched.  Replaces the candidate cache of
 * the reference's GPUMD evaluator (rune/mobius/src/mobius.cu:241-271,
 * :334-402: 1 A skin, reuse while every atom moved less than skin / 2, new
 * search on a box or pbc change). */
int rune_nlist_update(rune_nlist *nl, int64_t n_atoms, const double *d_positions,
                      int32_t n_structures, const int64_t *h_struct_ptr,
                      const double *h_cells, const int32_t *h_pbc,
                      double rc_radial, double rc_angular,
                      int32_t max_radial, int32_t max_angular, double skin,
                      void *stream, int64_t *n_records, int32_t *searched);

/* Records from the reference's padded batch tensors (-1 padded int64
 * [N,K] neighbour rows and fp32 [N,K,3] offsets, batch.py:9-39), with fp32
 * positions [N,3]; vec = (p[j] + offset) - p[i] as descriptor.py:813-817.
 * Radial and angular records are stored separately (radial first). */
int rune_nlist_from_padded(rune_nlist *nl, int64_t n_atoms, const float *d_positions,
                           const int64_t *d_radial_nbr, const float *d_radial_off,
                           int32_t k_radial, const int64_t *d_angular_nbr,
                           const float *d_angular_off, int32_t k_angular,
                           int32_t n_structures, const int64_t *h_struct_ptr,
                           void *stream, int64_t *n_records);

/* Copy the records into caller buffers (device; any pointer may be NULL):
 * ptr int32[N+1], view int32[N,4], nbr int32[E], shift int32[E,3],
 * vec float[E,4]. */
int rune_nlist_export(const rune_nlist *nl, int32_t *d_ptr, int32_t *d_view,
                      int32_t *d_nbr, int32_t *d_shift, float *d_vec, void *stream);

int64_t rune_nlist_atoms(const rune_nlist *nl);
int64_t rune_nlist_records(const rune_nlist *nl);

/* ------------------------------------------------------------------------
 * Models.
 *
 * Replaces load_model (rune/mobius/plugin.py:125-142, rune/nep/plugin.py:
 * 57-75): the handle is configured from the resolved model_params and then
 * receives every state_dict tensor by its reference name, like
 * load_state_dict(strict=True).
 * ---------------------------------------------------------------------- */
typedef struct rune_model rune_model;

enum { RUNE_FAMILY_MOBIUS = 0, RUNE_FAMILY_NEP = 1 };
enum { RUNE_ACT_TANH = 0, RUNE_ACT_SILU = 1, RUNE_ACT_GELU = 2 };
enum { RUNE_ZBL_NONE = 0, RUNE_ZBL_UNIVERSAL = 1, RUNE_ZBL_FLEXIBLE = 2 };
enum { RUNE_MESSAGE_SCALAR = 0, RUNE_MESSAGE_EQUIVARIANT = 1 };

typedef struct {
    int32_t family;            /* RUNE_FAMILY_*                                  */
    int32_t n_types;
    int32_t n_desc_radial;     /* n_max_radial + 1                               */
    int32_t k_radial;          /* basis_size_radial + 1                          */
    int32_t n_desc_angular;
    int32_t k_angular;
    int32_t l_max;
    int32_t has_q[6];          /* q222, q1111, q112, q123, q233, q134            */
    double rc_radial;
    double rc_angular;
    /* Möbius (rune/mobius/model.py:78-254) */
    int32_t hidden_dim;
    int32_t ffn_dim;
    int32_t blocks;
    int32_t activation;        /* RUNE_ACT_*                                     */
    int32_t message_layers;
    int32_t message_mode;      /* RUNE_MESSAGE_*                                 */
    int32_t message_dim;
    int32_t pair_dim;
    int32_t message_groups;
    int32_t vector_channels;
    int32_t message_basis_size;
    int32_t equivariant_channels;
    int32_t equivariant_l_max;
    double message_cutoff;
    double norm_eps;
    /* ZBL (rune/mobius/zbl.py:24-67, rune/nep/zbl.py) */
    int32_t zbl_mode;          /* RUNE_ZBL_*                                     */
    double zbl_rc_inner;
    double zbl_rc_outer;
    /* NEP4 (rune/nep/model.py:49-85): single hidden layer */
    int32_t nep_hidden;
    /* n_types element symbols in type order; resolves the per-element keys
     * "element_mlps.<symbol>...." of NEP state dicts (may be NULL for Möbius) */
    const char *const *elements;
} rune_model_config;

int rune_model_create(const rune_model_config *config, rune_model **out);
void rune_model_destroy(rune_model *model);

/* Hand over one state_dict tensor (fp32, C-contiguous, host memory) under its
 * reference key, e.g. "message_blocks.0.edge_mlp.0.weight". */
int rune_model_set_tensor(rune_model *model, const char *name, const float *h_data,
                          int64_t n_elements);

/* Check that every required tensor was given, pack and upload the weights. */
int rune_model_finalize(rune_model *model);

/* Create and finalize a model from its text artifact, so a C/C++ caller needs
 * no PyTorch pickle: "mobius1" files (rune/mobius/export.py:120-146, read and
 * validated as the GPUMD evaluator's read_model, rune/mobius/src/mobius.cu:
 * 26-151, with its messages) or "nep4" / "nep4_zbl" files (reader of
 * rune/nep/model.py:284-489; load_model of rune/nep/plugin.py:57-75 for
 * *.txt).  The weights equal those of the PyTorch loaders bit for bit. */
int rune_model_load(const char *path, rune_model **out);

/* Cutoffs of a model and, for models made by rune_model_load, the neighbour
 * limits its file names (0 for models made from a config).  Any output
 * pointer may be NULL.  (The reference reads them from model_params.) */
int rune_model_limits(const rune_model *model, double *rc_radial, double *rc_angular,
                      int32_t *max_radial, int32_t *max_angular);

/* Element symbol of type `type` (type ids follow the model's element order;
 * "" when out of range or when the model was created without symbols). */
const char *rune_model_element(const rune_model *model, int32_t type);

/* Energies, forces and virials: Mobius.forward / NEP.forward
 * (rune/mobius/model.py:307-393, rune/nep/model.py:87-155).
 * d_types int32 [N]; outputs (device, may be NULL when not wanted):
 *   d_energies  float [N]   per-atom energies
 *   d_energy    float [B]   per-structure energies
 *   d_forces    float [N,3]
 *   d_virial    float [B,9] per-structure virial W_ab = -sum_e g_a r_b
 *   d_atom_virial float [N,9] the same, attributed to neighbour atoms
 * The list must have been built with this model's cutoffs. */
int rune_model_compute(rune_model *model, const rune_nlist *nl, const int32_t *d_types,
                       int32_t compute_forces, int32_t compute_virial,
                       float *d_energies, float *d_energy, float *d_forces,
                       float *d_virial, float *d_atom_virial, void *stream);

/* Allocation-free evaluation.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * outputs and errors as rune_model_compute, but the workspace is a static
 * device array of rune_model_static_scratch_bytes() bytes (64 MiB) that every
 * GPU the library runs on holds until the process ends; the call allocates no
 * device memory.  An evaluation whose workspace exceeds the array fails with
 * RUNE_ERR_ARGUMENT before any launch (roughly: a few thousand atoms for
 * descriptor-only and NEP models, about 80 atoms of an OAM-EQ model).  All
 * calls on one GPU share the array and keep its last contents: calls that
 * overlap on one GPU (several streams or threads) race.  No phase timing is
 * recorded. */
int rune_model_compute_static(rune_model *model, const rune_nlist *nl, const int32_t *d_types,
                              int32_t compute_forces, int32_t compute_virial,
                              float *d_energies, float *d_energy, float *d_forces,
                              float *d_virial, float *d_atom_virial, void *stream);

/* Size in bytes of the static workspace of rune_model_compute_static. */
int64_t rune_model_static_scratch_bytes(void);

/* GPUMD-style per-atom outputs, accumulated (+=) in fp64 as GPUMD's
 * potentials do (rune/mobius/src/force.cu:47-84): d_potential [N];
 * d_force [3N] as three atom arrays x[0..N), y, z; d_virial [9N] as nine atom
 * arrays in the order xx, yy, zz, xy, xz, yz, yx, zx, zy of -r (x) g attributed
 * to the neighbour (the transpose of rune_model_compute's d_atom_virial).
 * Any output pointer may be NULL. */
int rune_model_compute_gpumd(rune_model *model, const rune_nlist *nl, const int32_t *d_types,
                             double *d_potential, double *d_force, double *d_virial,
                             void *stream);

/* 1 when the model supports GPUMD's heat-current / HNEMD observables (models
 * without message blocks: rune/mobius/src/mobius.cuh:18, the rejection of
 * rune/mobius/install_gpumd.py:38-46), else 0. */
int rune_model_supports_heat_current(const rune_model *model);

/* Width Q of the descriptor vector q: n_desc_radial + n_desc_angular * num_L
 * (the model's input_dim, rune/mobius/model.py:165). */
int32_t rune_model_input_dim(const rune_model *model);

/* Componentwise extrema of the raw descriptor values q (before q_scaler)
 * over the atoms of `nl`: the per-batch step of compute_descriptor_min_max
 * (rune/mobius/model.py:406-445, rune/nep/model.py:608-636) on the device.
 * d_q_min / d_q_max: float [Q] device; accumulate != 0 combines with the
 * values already there (the running min / max over batches), else they are
 * overwritten (+inf / -inf for an empty list).  NaN propagates as in
 * torch.amin / torch.minimum.  The scaler is then 1 / (max - min) where
 * max - min > 1e-12, else 1 (set_descriptor_scaler_from_min_max,
 * rune/mobius/model.py:446-465). */
int rune_model_descriptor_extrema(rune_model *model, const rune_nlist *nl,
                                  const int32_t *d_types, float *d_q_min, float *d_q_max,
                                  int32_t accumulate, void *stream);

/* Bytes of device workspace the handle currently holds. */
int64_t rune_model_workspace_bytes(const rune_model *model);

/* Phase timing.  rune_model_timing(model, mode): mode 1 makes
 * rune_model_compute record a HIP event on its stream at every phase boundary
 * (no synchronisation inside the call; the last 256 calls are kept) and
 * bracket every kernel-group launch (below); mode 2 brackets the group
 * launches only (no phase events, so a timed loop carries no per-phase
 * instrumentation); mode 0 turns both off.  rune_model_timing_read waits for
 * the phase events and returns the summed milliseconds per phase and the
 * number of calls.  (No counterpart in the reference; it feeds the roofline
 * measurement.) */
enum {
    RUNE_PHASE_DESCRIPTOR = 0,   /* K2 descriptor forward                       */
    RUNE_PHASE_DENSE_FWD = 1,    /* input projection + residual blocks           */
    RUNE_PHASE_MESSAGE_FWD = 2,  /* MP / EQ message blocks                       */
    RUNE_PHASE_READOUT = 3,      /* element heads (or NEP MLP, fwd + bwd)        */
    RUNE_PHASE_MESSAGE_BWD = 4,
    RUNE_PHASE_DENSE_BWD = 5,
    RUNE_PHASE_REVERSE = 6,      /* K3 descriptor reverse + ZBL                  */
    RUNE_PHASE_FORCES = 7,       /* K7 forces, virials, structure sums           */
    RUNE_N_PHASES = 8
};
int rune_model_timing(rune_model *model, int32_t enable);
int rune_model_timing_read(rune_model *model, double *ms_per_phase, int64_t *calls);

/* Kernel-group timing (no counterpart in the reference; it feeds the roofline
 * measurement).  While timing is on (mode 1 or 2), every launch of a group is bracketed
 * by two HIP events on the launch stream.  rune_model_timing_groups waits for
 * them and returns, per group, the summed milliseconds and the number of
 * launches since timing was enabled. */
enum {
    RUNE_GROUP_EDGE_GEMM = 0,     /* per-record MLP / gate GEMMs of MP and EQ blocks */
    RUNE_GROUP_EDGE_KERNELS = 1,  /* per-record message kernels (gather / transform /
                                     scatter, their reverse passes, edge preparation) */
    RUNE_N_GROUPS = 2
};
int rune_model_timing_groups(rune_model *model, double *ms_per_group, int64_t *launches);

#ifdef __cplusplus
}
#endif

#endif /* RUNE_HIP_H */
