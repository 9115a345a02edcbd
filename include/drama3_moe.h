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
  const void* gate_up_scale; /* bf16 scales (see formats) */
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
  uint32_t spin_limit;     /* bound on a workgroup's wait for another's result (0: default) */
  int32_t grid;            /* workgroups (0: as many as the device holds at once, capped by the work) */
  int32_t dn_start;        /* down weights load once this many 256ths of gate_up is done (0: at once) */
} d3_moe_a8_desc;

int64_t d3_moe_a8_workspace_bytes(int32_t M, int32_t topk, int32_t H, int32_t I);
int d3_moe_a8(const d3_moe_a8_desc* desc, void* stream);
/* Status word of a workspace after the launches on it completed: 0, or bit 0 if a wait hit spin_limit. Host pointer
 * `status` receives it (synchronous copy). */
int d3_moe_a8_status(const void* workspace, uint32_t* status);

/* ---- Checks of the A8 step (no reference counterpart: they expose the fused kernels' inner operations) --------
 * d3_gemv_a8_groups: rows [R, row_bytes(K)] of a bank in `format` against C <= 16 activation rows act [C, K] (int8;
 * e4m3 codes for F8). acc[R, K / 128, C]: the exact int32 dot product of each 128-column group (I8, W4, W6), or its
 * float value (F8, as float bits). R % 16 == 0, K % 512 == 0 or K % 128 == 0 as the format needs.
 * d3_unpack_rows: codes [R, K] int8 of W4 / W6 rows, in column order. */
int d3_gemv_a8_groups(int32_t format, const void* rows, int32_t R, int32_t K, const void* act, int32_t C, void* acc,
                      void* stream);
int d3_unpack_rows(int32_t format, const void* rows, int32_t R, int32_t K, void* codes, void* stream);

#ifdef __cplusplus
}
#endif
#endif
