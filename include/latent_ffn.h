/*
 * latent_ffn.h -- C ABI of the MI355X (gfx950) LATENT fused low-rank expert FFN.
 *
 * For every routed (token, slot) pair with expert e = ids[t][slot]:
 *
 *     y[t][slot] = ( SiLU(x[t] . A_g[e] . B_g[e]) * (x[t] . A_u[e] . B_u[e]) ) . A_d[e] . B_d[e]
 *
 * with the six factors dequantized on the fly from packed NF4 (per-32-group
 * fp16 scales) and optional per-group INT8 fallback, then either the
 * router-weighted sum over slots (LATENT_OUT_REDUCED) or the per-slot,
 * unweighted outputs of the ggml op (LATENT_OUT_PER_SLOT).
 *
 * Replaces, at the same boundary:
 *   - void ggml_cuda_latent_expert_ffn(ggml_backend_cuda_context&, ggml_tensor* dst)
 *       kernels/latent_fused_expert_ffn.h:64, implemented at
 *       kernels/latent_fused_expert_ffn.cu:134-292 (15 srcs, order at :135-149)
 *   - extern "C" __global__ latent_fused_expert_dispatch / latent_expert_reduce
 *       kernels/latent_fused_expert_ffn.h:61-62
 *   - swiglu_expert / load_pair of loader/latent_runtime.py:31-59 (Python side,
 *       bound through ctypes by latent_amd.runtime)
 *
 * Conventions
 *   - Plain pointers and sizes only.  All pointers are device pointers unless a
 *     comment says otherwise; the caller owns every buffer.
 *   - No call allocates device memory or synchronises the stream: scratch comes
 *     from the caller's workspace (size from latent_moe_workspace_size).
 *   - Errors are returned as LATENT_E_* status codes; nothing aborts.
 *   - Calls are stream ordered.  Concurrent calls on different streams must use
 *     different workspaces.
 *
 * Stacked operand layout (loader/write_latent_gguf.py:101-123, 227-257;
 * shapes of patches/002-latent-gguf-tensors.patch:135-148 with the packed code
 * axis asserted by tests/test_write_latent_gguf.py:112-154):
 *   gate_a, up_a : codes u8 [E][d ][R/2],  scales f16 [E][d ][R/32]
 *   gate_b, up_b : codes u8 [E][R ][ff/2], scales f16 [E][R ][ff/32]
 *   down_a       : codes u8 [E][ff][R/2],  scales f16 [E][ff][R/32]
 *   down_b       : codes u8 [E][R ][d/2],  scales f16 [E][R ][d/32]
 * Row-major, expert-major.  Low nibble = even column.  A group is 32
 * consecutive columns of one row.  Padding beyond an expert's true rank holds
 * zeros (code 7, scale 1.0), so computing over the padding changes nothing.
 */
#ifndef LATENT_FFN_H
#define LATENT_FFN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling in the HIP headers. */
typedef struct ihipStream_t* latent_stream_t;

/* ---- status codes ------------------------------------------------------- */
#define LATENT_OK 0
#define LATENT_E_INVALID (-1)     /* null pointer / inconsistent dims / bad enum */
#define LATENT_E_UNSUPPORTED (-2) /* valid request this build does not implement */
#define LATENT_E_WORKSPACE (-3)   /* workspace missing or smaller than required */
#define LATENT_E_HIP (-4)         /* a HIP runtime call or kernel launch failed */
#define LATENT_E_TIMEOUT (-5)     /* a bounded wait between workgroups expired: that call's output is undefined */

/* ---- element types ------------------------------------------------------ */
#define LATENT_F32 0
#define LATENT_F16 1
#define LATENT_BF16 2

/* ---- factor layouts ----------------------------------------------------- */
/* The stacked row layout above (loader/write_latent_gguf.py's). */
#define LATENT_LAYOUT_ROWS 0
/* The tile layout of the MFMA paths: every factor tensor, codes and scales
 * alike, reordered in place of the row layout by latent_tiles_repack (same
 * tensors, same sizes, each expert's bytes where its rows were). */
#define LATENT_LAYOUT_TILES 1

/* ---- factors, in the operand order (src3..src14 in code/scale pairs) ---- */
#define LATENT_GATE_A 0
#define LATENT_GATE_B 1
#define LATENT_UP_A 2
#define LATENT_UP_B 3
#define LATENT_DOWN_A 4
#define LATENT_DOWN_B 5

/* ---- output modes ------------------------------------------------------- */
/* f32 [T][d]: sum over slots of w*y (y when weight_before_down). */
#define LATENT_OUT_REDUCED 0
/* f32 [T][k][d]: per slot, unweighted unless weight_before_down, zero for a
 * dropped slot -- the dst of kernels/latent_fused_expert_ffn.cu:255-286. */
#define LATENT_OUT_PER_SLOT 1

/*
 * One stacked factor (codes + scales for all E experts).
 *   rows, cols      per-expert logical shape; cols % 32 == 0.
 *   expert stride   rows*cols/2 code bytes and rows*cols/32 scales.
 * Optional per-group INT8 fallback (no reference counterpart; the reference
 * only has whole-factor INT8 at group 64, loader/latent_loader.py:229-249):
 *   int8_bitmap     u32 [E][rows][ceil(cols/32/32)]; bit g => group g is INT8
 *   int8_row_offset i32 [E][rows]; index of the row's first INT8 group in data
 *   int8_data       i8  [n][32]; the flagged groups in (e,row,group) order
 * A flagged group's scale (absmax/127, fp16) sits in `scales`; its NF4 bytes
 * are ignored.  All three NULL => pure NF4.
 */
typedef struct latent_factor {
  const uint8_t* codes;
  const uint16_t* scales; /* IEEE binary16 bit patterns */
  const uint32_t* int8_bitmap;
  const int32_t* int8_row_offset;
  const int8_t* int8_data;
  int64_t rows;
  int64_t cols;
} latent_factor;

/*
 * Arguments of one MoE-layer expert FFN call: the 15 operands of
 * GGML_OP_LATENT_EXPERT_FFN (kernels/latent_fused_expert_ffn.cu:135-149) in
 * their order -- x, ids, weights, then gate_a..down_b with their scales --
 * plus the dimensions, per-expert ranks, output mode and workspace.
 */
typedef struct latent_moe_args {
  const void* x;            /* [T][d] of x_dtype (src0) */
  int32_t x_dtype;          /* LATENT_F32 | LATENT_F16 | LATENT_BF16 */
  const int32_t* ids;       /* [T][k] expert ids; id < 0 => dropped slot (src1) */
  const void* weights;      /* [T][k] router weights of weights_dtype (src2) */
  int32_t weights_dtype;    /* LATENT_F32 | LATENT_F16 */
  latent_factor gate_a, gate_b, up_a, up_b, down_a, down_b; /* src3..src14 */
  const int32_t* ranks;     /* [E][3] true (gate, up, down) ranks, or NULL => max_rank */
  int64_t n_tokens;         /* T */
  int64_t n_embd;           /* d */
  int64_t n_ff;             /* ff (per expert) */
  int64_t n_expert;         /* E */
  int64_t n_expert_used;    /* k, 1..64 */
  int64_t max_rank;         /* R, a multiple of 32 */
  int32_t weight_before_down;
  int32_t out_mode;         /* LATENT_OUT_REDUCED | LATENT_OUT_PER_SLOT */
  void* out;                /* f32, shape per out_mode */
  void* workspace;          /* device scratch, >= latent_moe_workspace_size() */
  size_t workspace_bytes;
  int32_t layout;           /* LATENT_LAYOUT_ROWS | LATENT_LAYOUT_TILES: how the 12 factor tensors are ordered */
} latent_moe_args;

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int latent_version(void);

/* Static text for a status code. */
const char* latent_status_string(int status);

/* Workspace bytes required by latent_moe_ffn_forward for these dims. */
int latent_moe_workspace_size(const latent_moe_args* args, size_t* bytes);

/*
 * The MoE-layer expert FFN (decode and prefill).  Stream ordered; ids outside
 * [0, E) are treated as dropped slots.  Replaces ggml_cuda_latent_expert_ffn
 * (kernels/latent_fused_expert_ffn.h:64).
 */
int latent_moe_ffn_forward(const latent_moe_args* args, latent_stream_t stream);

/*
 * latent_moe_ffn_forward without a caller workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * args->workspace and args->workspace_bytes are ignored: scratch comes from a
 * library-owned array of LATENT_NOALLOC_SCRATCH_BYTES on each GPU (held until
 * the process ends); a call whose latent_moe_workspace_size exceeds that
 * returns LATENT_E_WORKSPACE.  No call allocates.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams,
 * other host threads) race; calls in order on one stream do not.
 */
#define LATENT_NOALLOC_SCRATCH_BYTES (64u << 20)
#define LATENT_NOALLOC_CONTROL_BYTES (256u << 10)
int latent_moe_ffn_forward_noalloc(const latent_moe_args* args, latent_stream_t stream);

/*
 * 1 when this layer's factors can take LATENT_LAYOUT_TILES (pure NF4,
 * max_rank 256, n_embd and n_ff multiples of 256), 0 when not; reads only the
 * dimensions and the INT8 pointers.  No reference counterpart.
 */
int latent_tiles_supported(const latent_moe_args* args);

/*
 * Reorders one factor tensor pair between the row layout and the tile layout,
 * as a ggml backend repacks weights when it loads them (no reference
 * counterpart: the reference's kernels read the row layout,
 * kernels/latent_fused_expert_ffn.cu:17-18).  `factor` is LATENT_GATE_A ..
 * LATENT_DOWN_B; src and dst describe the same [n_expert][rows][cols] factor
 * (rows, cols as in the row layout; INT8 pointers NULL), src in the row
 * layout and dst in the tile layout when to_tiles != 0, the other way round
 * when 0.  Codes are repacked when both codes pointers are set, scales when
 * both scales pointers are (so a code tensor and its scale tensor can be
 * repacked on their own); the tile side must be 16-byte aligned and the two
 * sides must not overlap.  Shapes: gate_a, up_a, down_a rows % 256 == 0 and
 * cols == 256; gate_b, up_b rows == 256, cols % 128 == 0; down_b rows == 256,
 * cols % 256 == 0.  Expert e's bytes stay in expert e's byte range, so a
 * slice of experts repacks on its own.  Stream ordered; allocates nothing.
 */
int latent_tiles_repack(int32_t factor, const latent_factor* src, latent_factor* dst, int64_t n_expert,
                        int32_t to_tiles, latent_stream_t stream);

/*
 * Reads and clears the error word of a workspace.  A decode kernel whose
 * bounded wait for another workgroup expires sets it and finishes its work
 * on whatever data it has, so it always terminates; the output of that call
 * is undefined, and a late counter update may leave the workspace's control
 * block non-zero.  When the word is set this call therefore re-zeros the
 * whole control block (the first LATENT_NOALLOC_CONTROL_BYTES), after which
 * the workspace serves later calls correctly.  workspace == NULL (with
 * workspace_bytes == 0) checks the calling device's latent_moe_ffn_forward_noalloc
 * array instead.  Synchronises `stream`.  Returns LATENT_OK when no call on
 * this workspace timed out since the last check, LATENT_E_TIMEOUT when one
 * did.  No counterpart in the reference, whose kernels never wait on each
 * other.
 */
int latent_moe_check(void* workspace, size_t workspace_bytes, latent_stream_t stream);

/*
 * Which implementation latent_moe_ffn_forward uses for these arguments, the
 * first that supports the call in this order:
 *   2 = fp16-MFMA prefill: on average at least 16 routed pairs per active
 *       expert (or, for a layer in the tile layout, more routed pairs than
 *       path 3 takes), no INT8 groups, 16-byte aligned x; on the tile layout
 *       it streams 64-pair units of one expert, on the row layout (n_embd /
 *       n_ff / max_rank multiples of 128, n_ff and max_rank <= 2048, 16-byte
 *       aligned codes) it runs grouped GEMMs;
 *   3 = streaming fp16-MFMA decode: the factors are in the tile layout, 1 to
 *       4096 routed pairs, 16-byte aligned x;
 *   4 = multi-kernel fp16-MFMA path on the row layout, taken here when a
 *       factor has INT8 groups: at least 16 routed pairs, max_rank <= 512,
 *       16-byte aligned x (per-expert ranks allowed); factors decoded into
 *       LDS chunk by chunk;
 *   1 = single persistent fp32 decode kernel: row layout, 32 to 512 routed
 *       pairs, 2 * max_rank <= 1024, 16-byte aligned x (INT8 groups allowed);
 *   4 = as above, for the pure-NF4 calls path 1 does not take;
 *   0 = multi-kernel fp32 GEMV path: any call on the row layout.
 * A call in the tile layout that neither path 2 nor 3 takes is
 * LATENT_E_UNSUPPORTED.
 * < 0 = LATENT_E_* for bad arguments.  The environment variable
 * LATENT_MOE_PATH (general | fused | prefill | stream | rows) selects another path
 * that supports the call, for comparisons.
 * Diagnostic only; no counterpart in the reference.
 */
int latent_moe_path(const latent_moe_args* args);

/*
 * Launch style of a call that takes the streaming path (latent_moe_path 3):
 *   2 = small-batch chain: one launch for at most 32 routed pairs, every
 *       workgroup's tiles loaded first, grouping and combine inside (taken by
 *       default wherever a grid of at most four resident grids gives each
 *       workgroup tiles that fit its registers);
 *   0 = one launch per phase (the default otherwise; LATENT_STREAM_LAUNCH=phases
 *       also for small batches).
 * LATENT_E_UNSUPPORTED when the call does not take the streaming path.
 * Diagnostic only; no counterpart in the reference.
 */
int latent_stream_launch(const latent_moe_args* args);

/*
 * Dequantize expert `expert` of one stacked factor into f32 [rows][cols]
 * (out, device).  Bit-exact restatement of dequantize_nf4 / dequantize_int8
 * (loader/latent_loader.py:133-145, 161-170): one fp32 multiply per element.
 */
int latent_unpack(const latent_factor* factor, int64_t expert, float* out, latent_stream_t stream);

/*
 * Per-row NF4 pack of f32 [rows][cols] (device) into codes u8 [rows][cols/2]
 * and fp16 scales [rows][cols/32]; cols % 32 == 0.  Byte-identical to
 * quantize_nf4 per row (loader/latent_loader.py:111-130,
 * loader/write_latent_gguf.py:227-257).
 */
int latent_pack_nf4(const float* values, int64_t rows, int64_t cols, uint8_t* codes, uint16_t* scales,
                    latent_stream_t stream);

/*
 * INT8 pack of `n_groups` groups of 32 f32 values (device): q i8 [n][32] and
 * fp16 scales [n].  Byte-identical to quantize_int8(group_size=32)
 * (loader/latent_loader.py:148-158).
 */
int latent_pack_int8(const float* values, int64_t n_groups, int8_t* q, uint16_t* scales, latent_stream_t stream);

/* ---- one expert on the reference's own factor artifacts ------------------ */
#define LATENT_Q_NF4 0
#define LATENT_Q_INT8 1

/*
 * One factor as loader/latent_loader.py stores it (NPZ keys
 * <name>.{a,b}.{nf4|int8,scales,shape}, :253-260): the logical [rows][cols]
 * matrix flattened row-major and quantized in groups of group_size
 * consecutive flat elements, so a group may straddle rows.
 *   LATENT_Q_NF4   data u8 [ceil(rows*cols/2)], two codes per byte, low
 *                  nibble = even flat index (quantize_nf4, :111-130)
 *   LATENT_Q_INT8  data i8 [groups*group_size] (quantize_int8, :148-158)
 *   scales         f16 [groups], groups = ceil(rows*cols/group_size)
 * group_size must be a power of two (the reference runtime reads NF4 at 32
 * and INT8 at 64, loader/latent_runtime.py:25-27).
 */
typedef struct latent_flat_factor {
  const void* data;
  const uint16_t* scales; /* IEEE binary16 bit patterns */
  int32_t kind;           /* LATENT_Q_NF4 | LATENT_Q_INT8 */
  int32_t group_size;
  int64_t rows;
  int64_t cols;
} latent_flat_factor;

/*
 * Arguments of one single-expert SwiGLU FFN call:
 *   out = (SiLU(x.A_g.B_g) * (x.A_u.B_u) [* weight]) . A_d . B_d
 * with gate_a [d][r_g], gate_b [r_g][ff], up_a [d][r_u], up_b [r_u][ff],
 * down_a [ff][r_d], down_b [r_d][d]; the three ranks may differ.  `weight`
 * is applied only when weight_before_down is set and ignored otherwise, as in
 * the reference.
 */
typedef struct latent_expert_args {
  const float* x; /* [T][d] f32 */
  latent_flat_factor gate_a, gate_b, up_a, up_b, down_a, down_b;
  int64_t n_tokens; /* T */
  float weight;
  int32_t weight_before_down;
  float* out;      /* [T][d] f32 */
  void* workspace; /* device scratch, >= latent_expert_workspace_size() */
  size_t workspace_bytes;
} latent_expert_args;

/* Workspace bytes required by latent_expert_forward for these dims. */
int latent_expert_workspace_size(const latent_expert_args* args, size_t* bytes);

/*
 * swiglu_expert on load_pair'd factors (loader/latent_runtime.py:19-59): the
 * artifacts are dequantized on the fly exactly as dequantize_nf4 /
 * dequantize_int8 (loader/latent_loader.py:133-145, 161-170) decode them (one
 * fp32 multiply per element), and the chain runs in fp32.  Stream ordered;
 * allocates nothing.
 */
int latent_expert_forward(const latent_expert_args* args, latent_stream_t stream);

/* ---- router front end ---------------------------------------------------- */
/* Drop rules applied after top-k (dropped slot => id -1, weight 0; the kept
 * weights are not renormalised again). */
#define LATENT_DROP_NONE 0
/* Drop a slot whose renormalised weight is below drop_param. */
#define LATENT_DROP_BELOW 1
/* Keep the leading slots whose cumulative weight stays within drop_param of
 * the top-k total: adaptive_topk_inclusive / adaptive_topk_batch
 * (loader/adaptive_topk.py:29-90); drop_param in (0, 1]. */
#define LATENT_DROP_INCLUSIVE 2

/*
 * One router call.  Either logits = x . router (fp32 accumulation, summed over
 * 64-row slices of d in a fixed order) or caller logits (logits_in).  Then
 * softmax over the E experts, top-k by descending probability (ties -> lower
 * expert id), weights renormalised over the k kept slots, then the drop rule.
 * Produces the ids / weights operands of latent_moe_ffn_forward.
 */
typedef struct latent_route_args {
  const void* x;         /* [T][d] of x_dtype (unused when logits_in != NULL) */
  int32_t x_dtype;       /* LATENT_F32 | LATENT_F16 | LATENT_BF16 */
  const void* router;    /* [d][E] of router_dtype */
  int32_t router_dtype;  /* LATENT_F32 | LATENT_BF16 */
  const float* logits_in; /* [T][E] f32, or NULL => computed from x and router */
  float* logits_out;     /* [T][E] f32 written when not NULL */
  int32_t* ids;          /* [T][k] out; -1 for a dropped slot */
  float* weights;        /* [T][k] out */
  int64_t n_tokens;      /* T */
  int64_t n_embd;        /* d */
  int64_t n_expert;      /* E <= 1024 */
  int64_t n_expert_used; /* k <= 64 and <= E */
  int32_t drop_rule;     /* LATENT_DROP_* */
  float drop_param;
  void* workspace;       /* >= latent_route_workspace_size() bytes, device */
  size_t workspace_bytes;
} latent_route_args;

/* Workspace bytes required by latent_route (0 when logits_in is given). */
int latent_route_workspace_size(const latent_route_args* args, size_t* bytes);

/*
 * Router logits, softmax, top-k, renormalisation and drop on the device.
 * No counterpart kernel in the reference: routing belongs to the graph
 * builder there (build_moe_ffn_latent, README.md:111-113), and the drop rule
 * to loader/adaptive_topk.py:29-90.  Stream ordered; allocates nothing.
 */
int latent_route(const latent_route_args* args, latent_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* LATENT_FFN_H */
