/*
 * mko.h -- C ABI of the MI355X (gfx950) SSM scan library, libmko.so.
 *
 * Plain pointers and sizes only: no torch or C++ types cross this boundary.  Every
 * entry point takes a POD parameter block and a HIP stream (passed as void*, a
 * hipStream_t; NULL is the default stream), launches asynchronously on that
 * stream and returns MKO_OK or an error code; mko_last_error() then describes
 * the failure (thread-local).
 *
 * Ownership: the caller allocates every input, output and workspace; the
 * library never allocates or frees device memory (its one static device array,
 * behind mko_state_update_bwd_static, comes with the code object).  Inputs are
 * never written.
 * All tensors are dense row-major (contiguous) in the layouts documented per
 * field.  dtype fields take MKO_F32 / MKO_F16 / MKO_BF16 (and MKO_F64 for the SSD); every
 * kernel computes in float32 (float64 for float64 SSD inputs) and rounds once when it stores a
 * 16-bit output.
 *
 * The reference (dbydd/metal-kernelops) has no native ABI: its Python launches
 * Metal kernels through torch.mps.compile_shader.  Each entry point below names
 * the reference function it replaces (paths relative to src/metal_kernelops/).
 */
#ifndef MKO_H
#define MKO_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MKO_ABI_VERSION 1

/* MKO_F64 is taken by the SSD entry points only (mko_ssd_*), where every floating-point
 * array of the parameter block is then float64; the other entry points refuse it. */
enum mko_dtype { MKO_F32 = 0, MKO_F16 = 1, MKO_BF16 = 2, MKO_F64 = 3 };

enum mko_status {
  MKO_OK = 0,
  MKO_EINVAL = 1,       /* bad shape, pointer, dtype or flag */
  MKO_ELAUNCH = 2,      /* the HIP runtime refused a launch */
  MKO_EUNSUPPORTED = 3, /* valid request outside what the kernels implement */
  MKO_EWORKSPACE = 4    /* workspace missing or smaller than *_workspace_size() */
};

/* MKO_ABI_VERSION of the loaded library. */
int mko_abi_version(void);
/* Message for the last non-zero status returned on this thread ("" if none). */
const char* mko_last_error(void);
/* sizeof() of the parameter blocks, so a binding can check its mirror of them. */
size_t mko_sizeof_selscan_params(void);
size_t mko_sizeof_state_update_params(void);
size_t mko_sizeof_ssd_params(void);
size_t mko_sizeof_path_params(void);
size_t mko_sizeof_conv1d_params(void);
size_t mko_sizeof_conv1d_update_params(void);
size_t mko_sizeof_gated_norm_params(void);

/* Kernel timing (observability).  While enabled, every kernel the library
 * launches is bracketed by HIP events on its launch stream; the per-kernel totals
 * are resolved (synchronising on those events) when read.  No reference
 * counterpart: the reference times whole calls with wall clocks. */
int mko_profile_enable(int on);   /* returns the previous setting */
void mko_profile_reset(void);
int mko_profile_count(void);      /* number of distinct kernels timed */
int mko_profile_entry(int index, char* name, size_t name_len, double* total_ms, int64_t* launches);

/* Streaming device copy (measurement).  No reference counterpart: the reference's
 * verifiers time a state-sized torch copy as their floor (benchmarks/verify_mamba2_state.py:
 * 398-401, 431-445); this is the library's own, tuned for this part, so that the state
 * read-modify-write kernels are measured against the rate a read-and-write stream reaches
 * here.  Copies `bytes` from src to dst (16-byte aligned, not overlapping) on `stream`.
 * MKO_STREAM_NONTEMPORAL reads and writes with the nontemporal hint, as the decode kernels
 * read and write their state. */
#define MKO_STREAM_NONTEMPORAL 1u
int mko_stream_copy(const void* src, void* dst, size_t bytes, uint32_t flags, void* stream);

/* ======================================================================== */
/* Mamba-1 selective scan                                                     */
/* ======================================================================== */

#define MKO_SS_SOFTPLUS 1u /* delta = softplus(delta + delta_bias) (threshold 20) */

/* Steps between two saved scan states (the forward writes one state per 16
 * steps; the backward restarts its recompute of each 16-step block from them). */
#define MKO_SS_CHECKPOINT 16

typedef struct mko_selscan_params {
  /* forward inputs (also read by the backward) */
  const void* u;            /* (batch, dim, length)            u_dtype            */
  const void* delta;        /* (batch, dim, length)            delta_dtype, raw   */
  const float* A;           /* (dim, dstate)                   float32            */
  const void* B;            /* (batch, ngroups, dstate, length) bc_dtype          */
  const void* C;            /* (batch, ngroups, dstate, length) bc_dtype          */
  const float* D;           /* (dim,) or NULL                                     */
  const void* z;            /* (batch, dim, length) u_dtype, or NULL              */
  const float* delta_bias;  /* (dim,) or NULL                                     */
  /* forward outputs */
  void* out;                /* (batch, dim, length) u_dtype                        */
  float* states;            /* (batch, mko_selscan_num_checkpoints(length), dim, dstate):
                               the state entering every 16-step block, state-fastest;
                               written by the forward, read by the backward         */
  /* backward input */
  const void* dout;         /* (batch, dim, length) u_dtype                        */
  /* backward outputs (any may be NULL when that gradient is not wanted, except
     du and ddelta which are always written) */
  void* du;                 /* (batch, dim, length) u_dtype                        */
  void* ddelta;             /* (batch, dim, length) delta_dtype: grad of raw delta */
  float* dA;                /* (dim, dstate)                                       */
  void* dB;                 /* (batch, ngroups, dstate, length) bc_dtype           */
  void* dC;                 /* (batch, ngroups, dstate, length) bc_dtype           */
  float* dD;                /* (dim,), needs D                                     */
  void* dz;                 /* (batch, dim, length) u_dtype, needs z               */
  float* ddelta_bias;       /* (dim,), needs delta_bias                            */
  void* workspace;
  size_t workspace_bytes;
  int64_t batch, dim, length, dstate, ngroups;
  int32_t u_dtype, delta_dtype, bc_dtype;
  uint32_t flags;
} mko_selscan_params;

/* ceil(length / MKO_SS_CHECKPOINT): the second extent of params.states. */
int64_t mko_selscan_num_checkpoints(int64_t length);

/* Replaces _Scan.forward (scan.py:237-255) together with the pointwise pre/post
 * ops of selective_scan (scan.py:311-319): out = (scan(u, softplus(delta +
 * delta_bias), A, B, C) + u*D) * silu(z), each stage optional as in the
 * reference.  dstate <= 32 (the reference kernels assume the same). */
size_t mko_selscan_fwd_workspace_size(const mko_selscan_params* p);
int mko_selscan_fwd(const mko_selscan_params* p, void* stream);

/* Replaces _Scan.backward (scan.py:257-280) and the autograd of the pre/post
 * ops: given dout and the forward's inputs and states, writes the gradients
 * listed above.  Every sum (dB/dC over channels, dA/dD/ddelta_bias over batch and
 * time) runs in a fixed order, so repeated runs are bit-identical. */
size_t mko_selscan_bwd_workspace_size(const mko_selscan_params* p);
int mko_selscan_bwd(const mko_selscan_params* p, void* stream);

/* Which mapping each direction takes for this geometry, from the sizes alone (a call
 * still falls back to the lane-per-channel kernels when B/C rows are not 16-byte
 * aligned): 1 for the lane-per-(channel, state) kernels, 0 for the lane-per-channel ones.
 * Host only, no launch; pointers are not read.  No reference counterpart (the reference
 * has one Metal mapping). */
int mko_selscan_plan(const mko_selscan_params* p, int* fwd_lane, int* bwd_lane);

/* ======================================================================== */
/* Mamba-2 decode state update                                                */
/* ======================================================================== */

#define MKO_SU_SOFTPLUS 1u   /* delta = softplus(dt + dt_bias) */
#define MKO_SU_DT_PER_ROW 2u /* dt is (batch, nheads, headdim) instead of (batch, nheads) */
#define MKO_SU_D_PER_ROW 4u  /* D is (nheads, headdim) instead of (nheads,) */

typedef struct mko_state_update_params {
  const void* state;        /* (batch, nheads, headdim, dstate) state_dtype        */
  const void* x;            /* (batch, nheads, headdim)        x_dtype             */
  const void* dt;           /* (batch, nheads) or (batch, nheads, headdim) dt_dtype */
  const float* A;           /* (nheads,)                                           */
  const void* B;            /* (batch, ngroups, dstate)        bc_dtype            */
  const void* C;            /* (batch, ngroups, dstate)        bc_dtype            */
  const float* D;           /* (nheads,) or (nheads, headdim), or NULL             */
  const void* z;            /* (batch, nheads, headdim) x_dtype, or NULL           */
  const float* dt_bias;     /* (nheads,) or NULL                                   */
  /* forward outputs */
  void* new_state;          /* (batch, nheads, headdim, dstate) state_dtype; may alias
                               state (in-place decode)                             */
  void* y;                  /* (batch, nheads, headdim) state_dtype                */
  /* backward inputs: upstream grads of y and new_state (either may be NULL) */
  const float* dy;          /* (batch, nheads, headdim) float32                    */
  const float* dnew_state;  /* (batch, nheads, headdim, dstate) float32            */
  /* backward outputs, float32 (dz/dD/ddt_bias only with z/D/dt_bias) */
  float* grad_state;        /* (batch, nheads, headdim, dstate)                    */
  float* dx;                /* (batch, nheads, headdim)                            */
  float* ddt;               /* shape of dt                                         */
  float* dA;                /* (nheads,)                                           */
  float* dB;                /* (batch, ngroups, dstate)                            */
  float* dC;                /* (batch, ngroups, dstate)                            */
  float* dD;                /* shape of D                                          */
  float* dz;                /* (batch, nheads, headdim)                            */
  float* ddt_bias;          /* (nheads,)                                           */
  void* workspace;
  size_t workspace_bytes;
  int64_t batch, nheads, headdim, dstate, ngroups;
  int32_t state_dtype, x_dtype, dt_dtype, bc_dtype;
  uint32_t flags;
} mko_state_update_params;

/* Replaces the Metal state_update_{f32,f16,bf16} kernel and _launch
 * (cv/mamba2_state.py:184-267, 601-637): one fused read-modify-write of the
 * state per decode step. */
int mko_state_update_fwd(const mko_state_update_params* p, void* stream);

/* Replaces _StateUpdate.backward (cv/mamba2_state.py:653-756) and its Metal
 * state_update_backward / state_update_reduce kernels (:269-536): every
 * gradient has one writer, so repeated runs are bit-identical. */
size_t mko_state_update_bwd_workspace_size(const mko_state_update_params* p);
int mko_state_update_bwd(const mko_state_update_params* p, void* stream);

/* Bytes of the static device array behind mko_state_update_bwd_static (one array per
 * GPU the library runs on, held until the process ends). */
#define MKO_SU_STATIC_SCRATCH_BYTES (32u << 20)

/* No counterpart in the reference: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving or training loops, harnesses that
 * forbid hipMalloc).  The backward of mko_state_update_bwd, with its per-head partials
 * in the library's static scratch array instead of p->workspace (ignored); it calls no
 * allocator.  The problem must need at most MKO_SU_STATIC_SCRATCH_BYTES of partials
 * (mko_state_update_bwd_workspace_size(p); config 5's 256 x 80 heads need 26.4 MB),
 * else MKO_EWORKSPACE.  The stream must belong to the current device.  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (two streams, or two
 * host threads) race.  Nothing in the array needs clearing between calls: each call
 * writes every partial it reads. */
int mko_state_update_bwd_static(const mko_state_update_params* p, void* stream);

/* ======================================================================== */
/* Mamba-2 SSD chunk scan                                                     */
/* ======================================================================== */

#define MKO_SSD_SOFTPLUS 1u  /* delta = softplus(dt + dt_bias) */
#define MKO_SSD_D_PER_ROW 2u /* D is (nheads, headdim) instead of (nheads,) */
#define MKO_SSD_SAVE_Y 4u    /* the forward also saves the chunk output before the skip and
                                the gate (fp32), so the backward need not recompute it; the
                                flag must be the same for the forward and its backward.  16-bit
                                inputs with dstate <= 128 ignore it: their backward always
                                recomputes that output, and mko_ssd_saved_bytes leaves it out */

typedef struct mko_ssd_params {
  const void* x;              /* (batch, length, nheads, headdim)  x_dtype            */
  const void* dt;             /* (batch, length, nheads)           dt_dtype, raw      */
  const float* A;             /* (nheads,)                                            */
  const void* B;              /* (batch, length, ngroups, dstate)  bc_dtype           */
  const void* C;              /* (batch, length, ngroups, dstate)  bc_dtype           */
  const float* D;             /* (nheads,) or (nheads, headdim), or NULL              */
  const void* z;              /* (batch, length, nheads, headdim) x_dtype, or NULL    */
  const float* dt_bias;       /* (nheads,) or NULL                                    */
  const void* initial_states; /* (batch, nheads, headdim, dstate) x_dtype, or NULL    */
  /* forward outputs */
  void* y;                    /* (batch, length, nheads, headdim) x_dtype             */
  void* final_state;          /* (batch, nheads, headdim, dstate) x_dtype             */
  void* saved;                /* mko_ssd_saved_bytes(): written by the forward, read by
                                 the backward (chunk states, step sums, C.B blocks)  */
  /* backward inputs */
  const void* dy;             /* (batch, length, nheads, headdim) x_dtype             */
  const void* dfinal;         /* (batch, nheads, headdim, dstate) x_dtype, or NULL    */
  /* backward outputs (dD/dz/ddt_bias/dinitial only with D/z/dt_bias/initial_states) */
  void* dx;                   /* x_dtype                                              */
  void* ddt;                  /* dt_dtype                                             */
  float* dA;                  /* (nheads,)                                            */
  void* dB;                   /* bc_dtype                                             */
  void* dC;                   /* bc_dtype                                             */
  float* dD;                  /* shape of D                                           */
  void* dz;                   /* x_dtype                                              */
  float* ddt_bias;            /* (nheads,)                                            */
  void* dinitial;             /* x_dtype                                              */
  void* workspace;
  size_t workspace_bytes;
  int64_t batch, length, nheads, headdim, ngroups, dstate;
  int32_t x_dtype, dt_dtype, bc_dtype;
  uint32_t flags;
} mko_ssd_params;

/* Size of the forward-to-backward save area (params.saved). */
size_t mko_ssd_saved_bytes(const mko_ssd_params* p);

/* Replaces mamba2_chunk_scan's composition and Metal forward
 * (cv/mamba2_chunk.py:447-533, 568-614, 617-678): y and the final state of the SSD
 * recurrence, computed in chunks with the intra-chunk, chunk-state and
 * state-to-output contractions on the matrix cores.  The result does not depend
 * on the caller's chunk_size; the kernels pick their own chunk (64 to 256).
 * float64 (x_dtype MKO_F64, which the reference's composition takes,
 * cv/mamba2_chunk.py:439-440): x, dt, B, C, z, initial_states and the outputs are float64
 * and so are A, D and dt_bias (and dA, dD, ddt_bias in the backward) despite the float*
 * field types; the per-token recurrence runs on the fp64 vector units, d_state <= 256. */
size_t mko_ssd_fwd_workspace_size(const mko_ssd_params* p);
int mko_ssd_fwd(const mko_ssd_params* p, void* stream);

/* Replaces the torch autograd of that composition (the reference has no
 * hand-written SSD backward): gradients of every differentiable input.  For 16-bit and
 * float32 inputs part of the work runs on a second stream of the current device that the
 * library creates on first use (non-blocking, default priority, kept until the process
 * ends); `stream` waits for it before the call's last kernel, so the outputs and the
 * workspace are ordered on `stream` alone.  While `stream` is being captured into a graph
 * everything runs on `stream`.  The stream must belong to the current device. */
size_t mko_ssd_bwd_workspace_size(const mko_ssd_params* p);
int mko_ssd_bwd(const mko_ssd_params* p, void* stream);

/* ======================================================================== */
/* Four-path 2D scan layout (VMamba's ss2d, cv/path_scan.py)                  */
/* ======================================================================== */

/* A (batch, rows, height, width) map is read along four paths; path k visits pixel
 * pos_k(i) at step i of L = height * width:
 *   k = 0: i      k = 1: (i % height) * width + i / height (down each column)
 *   k = 2: L-1-i  k = 3: pos_1(L-1-i)
 * rows is the channel count of u/dt/dy, or groups * dstate of B/C.  The 2D scan is
 * the Mamba-1 scan (mko_selscan_fwd/bwd) over the stacked layout, with dim and
 * ngroups four times the map's. */
typedef struct mko_path_params {
  const void* src;
  void* dst;
  int64_t batch, rows, height, width;
  int32_t dtype; /* of src and dst */
  float scale;   /* multiplies every output */
} mko_path_params;

/* src (batch, rows, L) -> dst (batch, 4 * rows, L):
 *   dst[b][k * rows + r][i] = scale * src[b][r][pos_k(i)].
 * Replaces _stack_spatial / _stack_groups (cv/path_scan.py:165-188), with the state
 * transpose of the Metal transpose_states kernel (:267-282) left to the scan's own
 * layout pass. */
int mko_path_stack(const mko_path_params* p, void* stream);

/* src (batch, 4 * rows, L) in step order -> dst (batch, rows, L) per pixel:
 *   dst[b][r][pix] = scale * ((s0 + s2) + (s1 + s3)), s_k = src[b][k * rows + r][step_k(pix)]
 * with step_k the inverse of pos_k.  Replaces merge_paths (cv/path_scan.py:380-404),
 * in its permuting form; the reference's forward merges per-pixel slices, this
 * build's forward merges step-ordered ones like its backward. */
int mko_path_merge(const mko_path_params* p, void* stream);

/* ======================================================================== */
/* Causal depthwise conv1d (cv/causal_conv1d.py)                              */
/* ======================================================================== */

#define MKO_CONV_SILU 1u /* out = silu(pre) instead of pre */

/* With z = cat(initial_state or zeros(width-1), x) along time:
 *   out[b][c][t] = act(bias[c] + sum_{j < width} weight[c][j] * z[b][c][t + j])
 *   final_state  = z[..., length : length + width - 1]
 * Every tensor is contiguous and of `dtype`; arithmetic is float32. */
typedef struct mko_conv1d_params {
  const void* x;             /* (batch, channels, length) */
  const void* weight;        /* (channels, width), width <= 32 */
  const void* bias;          /* (channels,) or NULL */
  const void* initial_state; /* (batch, channels, width - 1) or NULL (zeros) */
  void* out;                 /* forward: (batch, channels, length) */
  void* final_state;         /* forward: (batch, channels, width - 1), written when non-NULL */
  const void* dout;          /* backward: (batch, channels, length) */
  void* dx;                  /* backward: (batch, channels, length) */
  void* dweight;             /* backward: (channels, width) or NULL */
  void* dbias;               /* backward: (channels,) or NULL */
  void* dinitial;            /* backward: (batch, channels, width - 1) or NULL */
  void* workspace;           /* backward, when dweight or dbias: mko_conv1d_bwd_workspace_size() */
  size_t workspace_bytes;
  int64_t batch, channels, length, width;
  int32_t dtype;
  uint32_t flags;            /* MKO_CONV_SILU */
} mko_conv1d_params;

/* Replaces the Metal causal_conv1d_fwd kernel and _forward_metal
 * (cv/causal_conv1d.py:79-160, 533-549). */
int mko_conv1d_fwd(const mko_conv1d_params* p, void* stream);
/* Replaces _CausalConv1d.backward with the Metal causal_conv1d_bwd and
 * causal_conv1d_dwfinal kernels (cv/causal_conv1d.py:161-338, 562-607): dx, dinitial,
 * and dweight/dbias reduced over batch and time in a fixed order.  The gradient through
 * final_state is the caller's (it is a slice of cat(initial_state, x)). */
size_t mko_conv1d_bwd_workspace_size(const mko_conv1d_params* p);
int mko_conv1d_bwd(const mko_conv1d_params* p, void* stream);

/* Decode: x (batch, channels, q) advances a rolling state (batch, channels, span),
 * span >= width - 1, element (b, c, i) at b * state_stride_b + c * state_stride_c + i
 * (a slice of a larger cache).  out (batch, channels, q) is the convolution of
 * cat(state, x) at the q new tokens; state becomes cat(state, x)[..., q : q + span].
 * Replaces the Metal causal_conv1d_update kernel (cv/causal_conv1d.py:340-390, 690-756). */
typedef struct mko_conv1d_update_params {
  const void* x;
  void* state;
  const void* weight; /* (channels, width) */
  const void* bias;   /* (channels,) or NULL */
  void* out;
  int64_t batch, channels, q, span, width, state_stride_b, state_stride_c;
  int32_t dtype; /* of every tensor */
  uint32_t flags;
} mko_conv1d_update_params;

int mko_conv1d_update(const mko_conv1d_update_params* p, void* stream);

/* ======================================================================== */
/* Gated RMSNorm (cv/gated_norm.py)                                          */
/* ======================================================================== */

/* Where silu(z) enters; the numbering of the reference's _GATE_* constants
 * (cv/gated_norm.py:63-66). */
#define MKO_GATE_NONE 0   /* no z */
#define MKO_GATE_BEFORE 1 /* norm_before_gate=False: x' = x * silu(z) is normalised */
#define MKO_GATE_AFTER 2  /* norm_before_gate=True: the normalised output is multiplied by silu(z) */

/* Per (row, group) of `group` consecutive features:
 *   x'  = x * silu(z) (MKO_GATE_BEFORE) or x
 *   r   = 1 / sqrt(mean(x'^2) + eps)                       (biased mean over the group)
 *   out = (x' * r * weight + bias) * silu(z) (MKO_GATE_AFTER), or without the gate
 * x, z, out, dout, dx and dz are (rows, features) of `dtype`; weight and bias are
 * (features,) of `wdtype`; rstd, dweight and dbias are float32.  Arithmetic is float32. */
typedef struct mko_gated_norm_params {
  const void* x;
  const void* z;        /* NULL with MKO_GATE_NONE */
  const void* weight;   /* (features,) */
  const void* bias;     /* (features,) or NULL */
  void* out;            /* forward */
  float* rstd;          /* (rows, features / group): the forward writes it when non-NULL, the backward reads it */
  const void* dout;     /* backward */
  void* dx;             /* backward */
  void* dz;             /* backward, with a gate */
  float* dweight;       /* backward: (features,), summed over rows, or NULL */
  float* dbias;         /* backward: (features,), summed over rows, or NULL */
  void* workspace;      /* backward: mko_gated_norm_bwd_workspace_size() bytes */
  size_t workspace_bytes;
  int64_t rows, features, group; /* group divides features */
  float eps;
  int32_t dtype;        /* of x, z, out, dout, dx, dz */
  int32_t gate;         /* MKO_GATE_* */
  int32_t wdtype;       /* of weight and bias */
} mko_gated_norm_params;

/* Replaces the Metal fwd_* / fwd_stream_* kernels and _GatedRMSNorm.forward
 * (cv/gated_norm.py:154-183, 252-281, 565-604). */
int mko_gated_norm_fwd(const mko_gated_norm_params* p, void* stream);
/* Replaces _GatedRMSNorm.backward with the Metal bwd_*, bwd_c1_* and bwd_apply_*
 * kernels and the partial sums (cv/gated_norm.py:185-250, 283-340, 606-645): dx, dz,
 * and dweight/dbias reduced over rows in a fixed order. */
size_t mko_gated_norm_bwd_workspace_size(const mko_gated_norm_params* p);
int mko_gated_norm_bwd(const mko_gated_norm_params* p, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MKO_H */
