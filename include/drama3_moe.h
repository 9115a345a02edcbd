/* drama3_moe.h - C ABI of the MI355X (gfx950) routed-expert MoE library, libdrama3_moe.so.
 *
 * Plain pointers (device memory unless stated), 32/64-bit integers and a HIP stream passed as void*. Every call is
 * stream-ordered on `stream`, allocates nothing and waits on nothing on the host, so it can be captured in a HIP
 * graph. Return value: 0 on success, D3_EINVAL for arguments the kernels cannot take (the message is in
 * d3_last_error()), or a hipError_t (positive) from the launch.
 *
 * The reference binds its kernels through NVRTC (drama3/kernels.py:593-601: _kernel/_launch, launched on
 * torch.cuda.current_stream). Each entry point below names the reference kernel or Python function it replaces.
 */
#ifndef DRAMA3_MOE_H
#define DRAMA3_MOE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define D3_EINVAL (-1)

/* Weight formats of the A8 banks (fused layer, d3_moe_a8). A bank is [E * N, row_bytes] with its scales:
 *   D3_FMT_I8  int8 rows, bf16 scale per row                  scales [E * N]
 *   D3_FMT_W4  signed int4, 2 per byte along K, bf16 scale per 128-column group   scales [E * N, K / 128]
 *   D3_FMT_W6  signed 6-bit, 16 per 12 bytes along K, bf16 scale per 128-column group
 *   D3_FMT_F8  float8 e4m3fn rows, bf16 scale per row
 * Activations are quantized per row inside the kernels: int8 (absmax / 127) for I8, W4, W6; e4m3 (absmax / 448) for F8. */
enum { D3_FMT_I8 = 0, D3_FMT_W4 = 1, D3_FMT_W6 = 2, D3_FMT_F8 = 3 };

const char* d3_last_error(void);
int d3_version(void);

/* ---- Fused MoE layer for A8 banks ---------------------------------------------------------------------------
 * Replaces, for one layer and M rows (decode lines batched together), kernels.route + offload.resident_decode
 * (drama3/model.py:107-124 -> drama3/offload.py:108-123, which launch route_experts, rotate_rows, gemv_*, rotate_rows
 * and weighted_sum, kernels.py:39-76,222-314,466-536) and the row-by-row loop over batched lines (model.py:111-113):
 *   ids, w = top-k softmax of logits[m] (renormalized over the k, rounded to bf16)
 *   out[m] = bf16( sum_j w[m, j] * down_e( SiLU(gate_e(x[m])) * up_e(x[m]) ) ),  e = ids[m, j]
 * with gate_up = bank [E * 2I, H] (gate rows first, then up rows) and down = bank [E * H, I]. */
typedef struct d3_moe_a8_desc {
  const void* x;           /* [M, H] bf16 */
  const void* logits;      /* [M, E] bf16 router logits */
  const void* gate_up;     /* [E * 2I, row_bytes(H)] packed weights */
  const void* gate_up_scale; /* bf16 scales (see formats); this and down_scale 16-byte aligned */
  const void* down;        /* [E * H, row_bytes(I)] */
  const void* down_scale;
  void* out;               /* [M, H] bf16 */
  int64_t* ids_out;        /* [M, topk] or NULL */
  float* weights_out;      /* [M, topk] or NULL */
  void* workspace;         /* d3_moe_a8_workspace_bytes(...) bytes; zeroed once before first use */
  int64_t workspace_bytes;
  int32_t format;          /* D3_FMT_* */
  int32_t M;               /* rows, 1..16 */
  int32_t H;               /* hidden size: 2048 */
  int32_t I;               /* expert FFN size: 512 or 768 */
  int32_t E;               /* experts per layer, <= 256 */
  int32_t topk;            /* <= 8 */
  uint32_t spin_limit;     /* polls a workgroup waits for another's result before computing it itself (0: default);
                            * the output is the same either way (see d3_moe_a8_status) */
  int32_t grid;            /* workgroups (0: as many as the device holds at once, capped by the work) */
  /* The block around the routed experts, SparseMoeBlock.forward (drama3/model.py:107-124), for one row (M = 1, grid
   * 0): with `router` the logits are computed in the launch, bf16(x . router[e]) (model.py:115), and `logits` may be
   * NULL; with the shared expert, out = bf16(experts + bf16(bf16(sigmoid(bf16(x . shared_gate))) * bf16(shared(x))))
   * as model.py:123 rounds it. NULL: not used. */
  const void* router;        /* [E, H] bf16 */
  void* logits_out;          /* [E] bf16 router logits, or NULL */
  const void* shared_gate_up;        /* [2I, row_bytes(H)]: one expert in the layer's format */
  const void* shared_gate_up_scale;
  const void* shared_down;           /* [H, row_bytes(I)] */
  const void* shared_down_scale;
  const void* shared_gate;           /* [H] bf16 (shared_expert_gate, one output) */
  /* One-row schedule (M = 1, grid 0): hidden units per gate_up workgroup, 8 or 16 (0: 8 when the device holds k I / 8
   * workgroups at once, else 16). Both give the same output, bit for bit. */
  int32_t item_units;
  /* Test hook, never set in production: every wait for another workgroup's result gives up at once, as if the
   * producer never came, so every waiting workgroup computes what it waited for itself; the output must not change. */
  int32_t recompute_all;
} d3_moe_a8_desc;

int64_t d3_moe_a8_workspace_bytes(int32_t M, int32_t topk, int32_t H, int32_t I);
int d3_moe_a8(const d3_moe_a8_desc* desc, void* stream);
/* d3_moe_a8 without a caller's workspace, allocating nothing: no counterpart in the reference. For callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The workspace is a
 * static device array of the library, one per GPU, of 3,007,744 bytes: layers up to 16 rows, top-8, H 2048, I 768
 * (d3_moe_a8_workspace_bytes of the layer must fit, else D3_EINVAL). desc->workspace and workspace_bytes are ignored.
 * The first call on a device looks the array up; unless `stream` is capturing a graph it also clears the array with a
 * kernel on `stream` (the array starts zeroed when the library loads, so a first call under capture records no
 * clear). Every call on a GPU shares that GPU's array, which keeps the last call's contents. Calls must be ordered on
 * the device: on one stream, or across streams through an event dependency. Calls whose launches can overlap on the
 * device race on the array, host-ordered calls on two unordered streams included. */
int d3_moe_a8_noalloc(const d3_moe_a8_desc* desc, void* stream);
/* d3_moe_a8_status for the current device's static workspace of d3_moe_a8_noalloc (no counterpart in the reference;
 * for the same callers): the status bits since the last read, cleared. Synchronous; call it outside graph capture,
 * after the launches completed. Before any d3_moe_a8_noalloc call on the device it reports 0. */
int d3_moe_a8_noalloc_status(uint32_t* status);
/* Status bits of a workspace since the last call, after the launches on it completed (synchronous copies; the bits are
 * cleared): 0; bit 0 when a wait for another workgroup's result passed spin_limit and the waiting workgroup computed
 * the result itself (bit for bit what the producer would have published: the output is exact); bit 1 when a wait
 * still failed after that (that launch's output is not valid). Host pointer `status` receives them.
 * The workspace carries no state a launch must trust from an earlier one: its hand-off words are tagged with the
 * launch's epoch (dispatch ID plus a salt from the HSA queue's address), so it may move between streams, a graph
 * replayed on another stream included. Launches that overlap on one workspace race. */
int d3_moe_a8_status(void* workspace, uint32_t* status);

/* ---- The block for several rows (SparseMoeBlock.forward over a batch, drama3/model.py:107-124) -------------------
 * With d3_moe_a8 on all rows and a one-expert d3_moe_a8 for the shared expert, four launches run the block for M
 * rows, each over all of them:
 * d3_router_logits (model.py:115, self.gate(flat)): logits [M, E] bf16 = bf16(x . router[e]) with float sums in
 * the one-row block's order, so each row's logits equal what that block computes; x [M, H], router [E, H] bf16.
 * d3_block_combine (model.py:123): out[t] = bf16(routed[t] + bf16(gw_t * shared[t])), gw_t =
 * bf16(sigmoid(bf16(x[t] . gate))), as the one-row block's down blocks add the shared expert; routed, shared [M, H]
 * bf16 (the routed layer's output and the shared expert's, run as a layer of one expert at weight 1), gate [H] bf16.
 * H = 2048. */
int d3_router_logits(const void* x, const void* router, int32_t M, int32_t H, int32_t E, void* logits, void* stream);
int d3_block_combine(const void* x, const void* gate, const void* routed, const void* shared, int32_t M, int32_t H,
                     void* out, void* stream);

/* ---- MoE layer for many rows on A8 banks (prefill, many decode lines) --------------------------------------------
 * Replaces offload.resident_prefill (drama3/offload.py:139-149 -> grouped_int8 / grouped_fp8 / grouped_codes,
 * kernels.py:365-464,538-587) and FP8Experts.forward's prompt branch (offload.py:775-802) for A8 banks: the rows'
 * (row, expert) pairs are grouped by expert on the device (no host sync, unlike offload.py:142's bincount().tolist())
 * and each expert's weights are read once for all its rows by grouped MFMA products. Same layer as d3_moe_a8:
 *   out[t] = bf16( sum_j w[t, j] * down_e( SiLU(gate_e(x[t])) * up_e(x[t]) ) ),  e = ids[t, j]
 * Routing from logits (as d3_moe_a8) or given (ids_in [T, topk] int64 with weights_in [T, topk] float32, as
 * Experts.forward receives topk_idx / topk_weight, model.py:73). Several launches on `stream`; graph-capturable. */
typedef struct d3_moe_a8_prefill_desc {
  const void* x;             /* [T, H] bf16 */
  const void* logits;        /* [T, E] bf16, or NULL with ids_in / weights_in */
  const int64_t* ids_in;     /* [T, topk] */
  const float* weights_in;   /* [T, topk] */
  const void* gate_up;       /* A8 bank [E * 2I, row_bytes(H)] */
  const void* gate_up_scale;
  const void* down;          /* [E * H, row_bytes(I)] */
  const void* down_scale;
  void* out;                 /* [T, H] bf16 */
  int64_t* ids_out;          /* [T, topk] or NULL (routing from logits only) */
  float* weights_out;        /* [T, topk] or NULL */
  void* workspace;           /* d3_moe_a8_prefill_workspace_bytes(...) bytes; no initialization needed */
  int64_t workspace_bytes;
  int32_t format;            /* D3_FMT_* */
  int32_t T;                 /* rows */
  int32_t H;                 /* 2048 */
  int32_t I;                 /* 512 or 768 */
  int32_t E;                 /* experts, <= 1024 */
  int32_t topk;              /* <= 32 */
} d3_moe_a8_prefill_desc;

int64_t d3_moe_a8_prefill_workspace_bytes(int32_t T, int32_t topk, int32_t H, int32_t I, int32_t E);
int d3_moe_a8_prefill(const d3_moe_a8_prefill_desc* desc, void* stream);

/* ---- Checks of the A8 step (no reference counterpart: they expose the fused kernels' inner operations) --------
 * d3_gemv_a8_groups: rows [R, row_bytes(K)] of a bank in `format` against C <= 16 activation rows act [C, K] (int8;
 * e4m3 codes for F8). acc[R, K / 128, C]: the exact int32 dot product of each 128-column group (I8, W4, W6), or its
 * float value (F8, as float bits). R % 16 == 0, K % 512 == 0 or K % 128 == 0 as the format needs.
 * d3_unpack_rows: codes [R, K] int8 of W4 / W6 rows, in column order. */
int d3_gemv_a8_groups(int32_t format, const void* rows, int32_t R, int32_t K, const void* act, int32_t C, void* acc,
                      void* stream);
int d3_unpack_rows(int32_t format, const void* rows, int32_t R, int32_t K, void* codes, void* stream);
/* d3_cvt_fp8: float -> float8 e4m3fn codes (n a multiple of 4), by the hardware converter the kernels quantize with (hardware 1)
 * or the format-definition conversion (0); round to nearest, ties to even. */
int d3_cvt_fp8(const float* in, int32_t n, void* out, int32_t hardware, void* stream);

/* ---- Measurement of the device's ceiling (no reference counterpart) ---------------------------------------------
 * d3_stream_read: `grid` workgroups of 256 threads read `bytes` (a multiple of 16) at src once, 16 bytes a load;
 * nothing is written in practice (sink [1] receives a word only if the loads' xor equals a fixed constant). Timed
 * over a large buffer it gives the streaming HBM rate; over a layer's bytes, one launch's one-shot read time.
 * d3_empty_launch: a kernel of `grid` workgroups of 256 threads that does nothing: the fixed cost of a launch. */
int d3_stream_read(const void* src, int64_t bytes, uint32_t* sink, int32_t grid, void* stream);
int d3_empty_launch(int32_t grid, void* stream);

/* ---- FP8 weight with a bf16 scale per output row, bf16 activations ----------------------------------------------
 * The reference's CPU path for an FP8 weight, dequantize then multiply in bf16: nn.functional.linear(x,
 * dequantize_fp8(W, scale)) (drama3/offload.py:163-167 dequantize_fp8; the linear as experts_decode, offload.py:192-199,
 * and FP8Experts.forward's torch branch, offload.py:797-802, run it), with the scale per output row (absmax / 448)
 * instead of per 128 x 128 block:
 *   out[r, n] = bf16( sum_k x[r, k] * bf16(e4m3(weight[n, k]) * scale[n]) ),  float32 sums
 * x [rows, K] bf16 (rows 1..4, 16-byte aligned), weight [N, K] e4m3fn bytes, scale [N] bf16, out [rows, N] bf16;
 * K one of 512, 1024, 1536, 2048. Any N: k experts' rows stacked are one call (experts_decode's [k * 2I, H]). */
int d3_gemv_fp8_rows(const void* x, int32_t rows, const void* weight, const void* scale, void* out, int32_t N,
                     int32_t K, void* stream);

/* ---- The reference's own formats, one kernel per reference kernel (drama3/kernels.py SOURCE) -------------------
 * Float32 activations as in the reference. Slot-cache plans as there: plan [k, 2] int32 = (slot, code) per expert;
 * code 0 reads the slot fields, 1 reads the host (bank) fields and copies the expert into its slot when slot >= 0,
 * 2 (gemv_int8 only) is the CPU's: zeros, or with `late` the only experts run, from the host fields, when took_over[0].
 * "Host" fields may be device memory (an HBM-resident table: slot e = expert e and plan (e, 0)) or pinned host memory.
 * K is one of 256, 512, 768, 1024, 1536, 2048; N % 16 == 0 (N % 128 == 0 for FP8). */

/* route_experts (kernels.py:39-67, wrapper route kernels.py:647-653): per row of bf16 logits [rows, n] (n <= 1024),
 * ids [rows, k] int64 of the k (<= 32) largest in descending order (ties to the lower index) and weights [rows, k]
 * float32 = bf16(exp(l - l_max) / sum over the k). One wave per row. */
int d3_route(const void* logits, int32_t rows, int32_t n, int32_t k, int64_t* ids, float* weights, void* stream);

/* weighted_sum (kernels.py:69-76, wrapper kernels.py:656-661): out [H] bf16 = sum_e parts[e, h] * weights[e]. */
int d3_weighted_sum(const float* parts, const float* weights, int32_t k, int32_t H, void* out, void* stream);

/* rotate_rows (kernels.py:222-258, wrapper rotate kernels.py:636-644): mode 0 float rows [rows, K], 1 bf16 rows,
 * 2 SwiGLU of float [rows, 2K] gate | up; out [rows, K] float32 = rows times H256 on each 256 columns (K % 256 == 0).
 * Writes nothing unless only_if[0] (device int32) is non-zero. */
int d3_rotate(const void* x, int32_t mode, int32_t rows, int32_t K, float* out, const int32_t* only_if, void* stream);

/* gemv_int8 (kernels.py:260-314, wrapper kernels.py:664-671): out [k, N] float32 = (int8 row of the expert . x[e or 0])
 * * row scale, x [x_rows (1 or k), K] float32 (ConvRot basis); fields _qdata int8 [E * N, K], scale float32 [E * N]. */
int d3_gemv_int8(const float* x, int32_t x_rows, const int64_t* ids, const int32_t* plan, const int32_t* took_over,
                 int32_t late, void* slot_w, float* slot_s, const void* host_w, const float* host_s, float* out,
                 int32_t k, int32_t N, int32_t K, void* stream);

/* gemv_fp8 (kernels.py:316-363, wrapper kernels.py:674-681): out [k, N] = sum over columns of e4m3(W) * x * the
 * 128 x 128 block scale; fields weight uint8 [E * N, K], scale float32 [E * N / 128, K / 128]. The hardware e4m3fn
 * decode reads the NaN codes 0x7F / 0xFF as NaN (the reference's bit trick reads +-480). */
int d3_gemv_fp8(const float* x, int32_t x_rows, const int64_t* ids, const int32_t* plan, void* slot_w, float* slot_s,
                const void* host_w, const float* host_s, float* out, int32_t k, int32_t N, int32_t K, void* stream);

/* gemv_codes (kernels.py:466-536, wrapper kernels.py:703-713): W4A8 / W6A8 rows decoded to the int8 grid
 * (clamp(rint(value * e4m3 group scale), +-127), value = codebook[code] at 4 bits or code - 32 at 6 bits) . x, times
 * s_channel; fields _qdata uint8 [E * N, K * bits / 8] (nibble plane, then the 2-bit high planes at 6 bits), scale
 * e4m3 [E * N, K / 16], s_channel float32 [E * N]; codebook float32 [16] (4 bits) or NULL. */
int d3_gemv_codes(const float* x, int32_t x_rows, const int64_t* ids, const int32_t* plan, void* slot_w, void* slot_r,
                  float* slot_c, const void* host_w, const void* host_r, const float* host_c, const float* codebook,
                  int32_t bits, float* out, int32_t k, int32_t N, int32_t K, void* stream);

/* grouped_int8 / grouped_fp8 / grouped_codes (kernels.py:365-464,538-587, wrappers kernels.py:684-700,716-724):
 * kind 0 int8, 1 fp8, 4 / 6 codes. x [T, K] float32 rows sorted by expert; groups [n_groups, 5] int32 = (expert, slot,
 * fill, first row, rows); a group reads its slot, or the host fields when slot < 0 or fill (then copying the expert
 * into the slot). out [T, N] float32 rows of the groups (others untouched); a group with 0 rows reads nothing. The
 * products run on the vector unit in float32. */
int d3_grouped(int32_t kind, const float* x, const int32_t* groups, int32_t n_groups, void* slot_w, void* slot_s,
               void* slot_c, const void* host_w, const void* host_s, const void* host_c, const float* codebook,
               float* out, int32_t N, int32_t K, void* stream);

/* The same products on the matrix cores (same replacement, same fields and groups), for bank widths N % 64 == 0
 * (fp8: N % 128 == 0): d3_grouped_fp8 for fp8 banks on the bf16 cores, d3_grouped_i8 (below) for int8 and the codes
 * on the int8 cores. Both read the rows as planes [n_planes, plane] (plane a multiple of K: plane / K rows of K
 * elements per plane) and write out [rows, N]: row p of the groups' rows is the planes' row p (order NULL, rows <=
 * plane / K), or with order [rows] int64 the planes' row order[p] / k (a prompt's pairs read from its token rows,
 * no gathered copy; kept below plane / K). work: int32 device memory of d3_grouped_mfma_work_ints(n_groups, rows)
 * ints, filled by d3_grouped_plan (or d3_expert_groups) for these groups and rows (one plan serves both banks of a
 * layer): passes of up to 32 rows, a group whose rows lie outside [0, rows) skipped. fills_first: the groups' first
 * passes run first, then the others read a filled group from its slot, so an expert copied in crosses the bus once
 * however many rows it has.
 * d3_grouped_fp8's planes are bf16: bf16 rows as they are (n_planes 1), or float32 rows split into three bf16
 * planes by d3_split_bf16x3 (x [n] float32, n % 8 == 0 -> planes bf16 [3, n] = hi, mid, lo) or d3_prep_planes:
 * x == hi + mid + lo to within 2^-24 |x|, and every e4m3 weight is a bf16 value exactly, so each product is exact and
 * the sums float32, each 128-column chunk's scaled by its 128 x 128 block scale. */
int d3_split_bf16x3(const float* x, int64_t n, void* planes, void* stream);
int64_t d3_grouped_mfma_work_ints(int32_t n_groups, int64_t rows);
int d3_grouped_plan(const int32_t* groups, int32_t n_groups, int64_t rows, int32_t* work, int64_t work_ints,
                    void* stream);
int d3_grouped_fp8(const void* planes, int32_t n_planes, int64_t plane, const int64_t* order, int32_t k,
                   int32_t rows, const int32_t* groups, int32_t n_groups, const int32_t* work, int64_t work_ints,
                   int32_t fills_first, void* slot_w, void* slot_s, const void* host_w, const void* host_s,
                   float* out, int32_t N, int32_t K, void* stream);

/* A prompt's (token, k) pairs grouped by expert (offload.py:140-143, which sorts ids and counts each expert's pairs):
 * ids [P] int64 (P = T * k, row-major); order [P] int64 = the pairs' indices, each expert's pairs together and the
 * experts in ascending order; inverse [P] int32 = each pair's place in order (-1 for an id outside [0, E), which is
 * placed after every group); groups [E, 5] int32 = (e, e, 0, first, rows). Within a group the pairs' order is not
 * fixed: each output row of the grouped products depends on its own row alone. E <= 1024; one workgroup. work (or
 * NULL): the same launch also writes d3_grouped_plan's plan for these groups and P rows (work_ints >=
 * d3_grouped_mfma_work_ints(E, P)), which no later change of the groups' slot and fill fields alters. */
int d3_expert_groups(const int64_t* ids, int32_t P, int32_t E, int64_t* order, int32_t* inverse, int32_t* groups,
                     int32_t* work, int64_t work_ints, void* stream);

/* The planes d3_grouped_fp8 reads, from the rows themselves: planes bf16 [n_planes, P * K]; row p is x's row
 * order[p] / k (x's row p when order is NULL). mode 0: x float32 [., K]; 1: bf16 [., K]; 2: float32 gate | up
 * [., 2K] through SiLU(gate) * up (the SwiGLU between the banks, kernels.py:222-258). rotate: in the ConvRot basis
 * first (int8 and the codes; d3_rotate's transform). n_planes 3, or 1 for bf16 rows taken as they are (mode 1, no
 * rotation: the one plane holds them exactly). K in {256, 512, 768, 1024, 1536, 2048}. */
int d3_prep_planes(int32_t mode, int32_t rotate, int32_t n_planes, const void* x, const int64_t* order, int32_t k,
                   int32_t P, int32_t K, void* planes, void* stream);

/* The int8 formats' products (kind 0 int8, 4 / 6 codes; the same replacement: kernels.py:365-464,538-587 as called
 * from offload.py:126-149) on the int8 matrix cores. Their weights are integers |q| <= 127 before the row or channel
 * scale, so they enter the int8 products as bytes; the float32 rows enter as three int8 planes and a power-of-two row
 * scale S. d3_prep_planes_i8 takes the rows as d3_prep_planes does (mode, rotate, order, k) and writes planes int8
 * [3, P * K] = a0, a1, a2 and scales [P] float32: v / S = a0 + a1 / 254 + a2 / 254^2 + r with every a in
 * [-127, 127] and |r| < 0.5 / 254^2 + 2^-24, S the smallest power of two with max |v| <= 127 S, so the planes hold
 * each row to within 1.25e-7 of its largest magnitude, and rows of integers times a power of two exactly. A row
 * holding inf or NaN gets S = NaN (its products NaN), an all-zero row S = 0. d3_grouped_i8 reads those planes (plane
 * bytes per plane; rows, order, k, groups, work plan and fills_first as for d3_grouped_fp8; row p's scale is that of
 * the planes' row it reads); each plane's sums are exact int32, added in float32 at the end: out = scale * (S * (A0
 * + (A1 + A2 / 254) / 254)). N % 64 == 0. */
int d3_prep_planes_i8(int32_t mode, int32_t rotate, const void* x, const int64_t* order, int32_t k, int32_t P,
                      int32_t K, void* planes, float* scales, void* stream);
/* d3_expert_groups (work required) and d3_prep_planes_i8 over x's T token rows (mode 0 float32 or 1 bf16, order
 * NULL) in one launch, the grouping in its first workgroup and the rows in the others: a prompt's groups, plan,
 * planes and row scales with no launch between them (offload.py:138-143 and the first bank's rows). */
int d3_expert_groups_prep_i8(const int64_t* ids, int32_t P, int32_t E, int64_t* order, int32_t* inverse,
                             int32_t* groups, int32_t* work, int64_t work_ints, int32_t mode, int32_t rotate,
                             const void* x, int32_t T, int32_t K, void* planes, float* scales, void* stream);
int d3_grouped_i8(int32_t kind, const void* planes, const float* scales, int64_t plane, const int64_t* order,
                  int32_t k, int32_t rows, const int32_t* groups, int32_t n_groups, const int32_t* work,
                  int64_t work_ints, int32_t fills_first, void* slot_w, void* slot_s, void* slot_c,
                  const void* host_w, const void* host_s, const void* host_c, const float* codebook, float* out,
                  int32_t N, int32_t K, void* stream);

/* The weighted sum over k (offload.py:144-149): out [T, H] = sum over j in order of weights[t, j] *
 * sorted_out[inverse[t k + j]] in float32 (pairs with inverse -1 left out), stored as float32 / bf16 / fp16
 * (out_type 0 / 1 / 2); weights [T, k] bf16 (weights_bf16) or float32. H % 4 == 0. */
int d3_combine_rows(const float* sorted_out, const int32_t* inverse, const void* weights, int32_t weights_bf16,
                    int32_t T, int32_t k, int32_t H, void* out, int32_t out_type, void* stream);

/* resolve_experts (kernels.py:78-191, wrapper resolve kernels.py:617-625): the slot cache's lookup and eviction for
 * one decode row's experts ids [k] (int64, k <= 32) of `layer`, on the device. State (device memory, updated in
 * place): table [layers * experts] (slot, -1, or -2 - slot while the host copies into it), owner [count] (key or -1),
 * score / at [layers * experts] (decayed use count, as of step at), pending [count], clock [1] (passes), budget [2]
 * (reservations left this step, per layer), reads [3] (hits, GPU fills, CPU experts), step [1] (this layer's step).
 * share [1] float: the GPU's share of the missed experts with `cpu`. plan [k, 2] int32 out = (slot, code): 0 cached,
 * 1 read from the bank and fill the slot, 2 left to the CPU (slot reserved for the host's copy, or -1). One
 * workgroup. */
int d3_resolve(const int64_t* ids, int32_t k, int32_t layer, int32_t layers, int32_t experts, int32_t* table,
               int32_t* owner, float* score, int32_t* at, int32_t* pending, int32_t count, int32_t* clock,
               int32_t* budget, int32_t* plan, int32_t* reads, int32_t* step, const float* share, double half_life,
               int32_t cpu, double admit, void* stream);

/* await_cpu (kernels.py:193-220, wrapper kernels.py:628-633): when plan [k, 2] leaves experts to the CPU, waits up to
 * timeout_us for the host flag (pinned host memory) to reach step[0], then out [H] float32 = the host's bf16 result
 * (pinned host memory); a late host gives zeros and took_over[0] = 1 (the GEMVs' `late` launch then runs those
 * experts). Without CPU experts it returns at once (zeros, took_over 0). */
int d3_await_cpu(const int32_t* plan, int32_t k, const int32_t* flag, const int32_t* step, const void* result,
                 int32_t timeout_us, float* out, int32_t* took_over, int32_t H, void* stream);

/* resident_decode in two launches (offload.py:108-123, which launches rotate, gemv, rotate(SwiGLU), gemv and
 * weighted_sum): kind 0 int8 (ConvRot), 1 fp8, 4 / 6 codes; banks resident (expert e in slot e) with the fields of
 * d3_gemv_* (gu_c / dn_c: channel scales, codes only). x [H] bf16, ids [k] int64, weights [k] float32 (k <= 8),
 * gu [k, I] float32 scratch (the hidden rows SiLU(gate) * up), out [H] bf16. H 1024 or 2048, I 512, 768 or 1024. */
int d3_resident_decode(int32_t kind, const void* x, const int64_t* ids, const float* weights, int32_t k,
                       const void* gu_w, const void* gu_s, const float* gu_c, const void* dn_w, const void* dn_s,
                       const float* dn_c, const float* gu_codebook, const float* dn_codebook, float* gu, void* out,
                       int32_t H, int32_t I, void* stream);

/* kernels.route + resident_decode in two launches (kernels.py:39-67,647-653 route_experts / route, then
 * offload.py:108-123 as d3_resident_decode): the row's routing runs in the gate_up launch's prologue, from the router's
 * logits [n] bf16 (k <= n <= 256), with route's key order and bf16-rounded softmax weights. ids [k] int64 and
 * weights [k] float32 are outputs (equal to d3_route's for the same logits); the other arguments as for
 * d3_resident_decode. */
int d3_resident_decode_routed(int32_t kind, const void* x, const void* logits, int32_t n, int32_t k, int64_t* ids,
                              float* weights, const void* gu_w, const void* gu_s, const float* gu_c, const void* dn_w,
                              const void* dn_s, const float* dn_c, const float* gu_codebook, const float* dn_codebook,
                              float* gu, void* out, int32_t H, int32_t I, void* stream);

/* resident_decode in one launch (offload.py:108-123, and with `logits` the routing of kernels.py:39-67 as
 * d3_resident_decode_routed does it): the same output, ids and weights as the two-launch entries, bit for bit. Each
 * gate_up workgroup hands its hidden units to the down workgroups of the same launch through `workspace`
 * (d3_resident_workspace_bytes(k, I) bytes, 256-byte aligned, zeroed once before first use; its words carry the
 * launch's epoch, so it needs no clearing between launches, on any stream). logits NULL: ids [k] and weights [k] are
 * inputs; else outputs. H 2048, I 512 or 768. spin_limit: polls a down workgroup waits for a hidden row before it
 * computes the row itself (0: default; the output is the same either way, see d3_resident_status). block_rows: output
 * rows per down workgroup, 4 or 8 (0: 4). recompute_all (test hook): every down workgroup computes the hidden rows
 * itself. Launches that overlap on one workspace race. */
int64_t d3_resident_workspace_bytes(int32_t k, int32_t I);
int d3_resident_decode_fused(int32_t kind, const void* x, const void* logits, int32_t n, int32_t k, int64_t* ids,
                             float* weights, const void* gu_w, const void* gu_s, const float* gu_c, const void* dn_w,
                             const void* dn_s, const float* dn_c, const float* gu_codebook, const float* dn_codebook,
                             void* workspace, int64_t workspace_bytes, uint32_t spin_limit, int32_t block_rows,
                             int32_t recompute_all, void* out, int32_t H, int32_t I, void* stream);
/* Status bits of a resident workspace since the last call, after its launches completed (synchronous copies; the bits
 * are cleared): 0, or bit 0 when a down workgroup stopped waiting and computed the hidden rows itself (the output is
 * exact either way). */
int d3_resident_status(void* workspace, uint32_t* status);

/* Check of the W4A8 / W6A8 decode on its own (kernels.py:466-483 decode_codes; no entry point of its own there):
 * codes [R, K] int8 of rows [R, K * bits / 8] with scales [R, K / 16]; K % 32 == 0. bits 4 or 6 decode as the GEMVs
 * and grouped products do; bits D3_DECODE_TABLE_W4 decodes 4-bit rows through the per-scale-byte tables the resident
 * decode kernels use. */
#define D3_DECODE_TABLE_W4 0x104
int d3_decode_codes(int32_t bits, const void* rows, const void* scales, const float* codebook, int32_t R, int32_t K,
                    void* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif
