/* pto_fuser_hip.h — C ABI of the MI355X (gfx950) delta-rule forward library, libptofuser_hip.so.
 *
 * This is the drop-in boundary for pto-fuser's chunked delta-rule forward.  The reference
 * hosts its fused kernels as ctypes-bound `.so` recipes (src/pto_fuser/fused.py:83-162) and its
 * triangular inverse as an opaque kernel (src/pto_fuser/registry.py:96-127); every entry point
 * below replaces one of those bindings.  Conventions, all plain C:
 *   - pointers are device pointers (HBM) unless stated; layouts are row-major and contiguous;
 *   - `dtype` selects the element type of the q/k/v/w/u operands: PF_DTYPE_F32 or PF_DTYPE_BF16;
 *     gates (g, beta, decay) are always fp32, outputs are fp32 unless stated;
 *   - `stream` is a hipStream_t passed as void* (torch.cuda.current_stream().cuda_stream);
 *     every *_exec only enqueues on that stream: no allocation, no host synchronisation, so it
 *     is capturable by a HIP graph (the reference's requirement, fused.py:5-9,96-100);
 *   - every *_exec returns an int status: PF_OK, a negative PF_ERR_* for a contract violation
 *     detected on the host (nothing is launched), or a positive hipError_t from the launch.
 *     The reference's execs return void (scan_lib.cpp:90, kkt_fused_lib.cpp:105).
 *   - *_setup returns an opaque workspace handle owned by the library (NULL on failure) and
 *     *_teardown frees it (scan_lib.cpp:81-99 discipline: allocate once, launch many).
 */
#ifndef PTO_FUSER_HIP_H
#define PTO_FUSER_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PF_DTYPE_F32 0
#define PF_DTYPE_BF16 1

#define PF_OK 0
#define PF_ERR_ARG (-1)       /* shape, dtype or null-pointer contract violated */
#define PF_ERR_WORKSPACE (-2) /* workspace handle missing or too small for this call */
#define PF_ERR_ALLOC (-3)     /* setup could not allocate its workspace */
#define PF_ERR_SCRATCH (-4)   /* input larger than the static scratch of pf_gdn_exec_static */

/* Human-readable text for a status code (static storage). */
const char* pf_status_string(int status);
/* ABI revision of this library. */
int pf_abi_version(void);
/* Hash of the sources, headers and compiler flags the library was built from (16 hex digits);
 * the Python loader refuses a library whose hash differs from the source tree's.  No counterpart
 * in the reference, whose registry recompiles per shape (fused.py:58-77). */
const char* pf_source_hash(void);

/* ------------------------------------------------------------------------------------------
 * Fused gated delta-rule forward (GDN; DeltaNet when g == NULL).
 * Replaces the lowered compiled_forward path of examples/attention/gdn.py:75-88: the
 * kkt_gated_native_v2 FusedNode (fused.py:500-517), the tri_inv_rec_unroll OpaqueNode
 * (registry.py:107-127), the two WY einsums (_gdn_full.py:199-200), the chunk_h_scan FusedNode
 * (fused.py:168-182, scan_lib.cpp:81-99) and the qkv_flash_native_v2 FusedNode
 * (fused.py:353-395, qkv_fused_lib.cpp:148-165), with the host coefficient prep of
 * prepare_gdn_bindings (_gdn_full.py:103-144) folded in.  Math: gdn_reference
 * (_gdn_full.py:57-97) plus an initial state h0 and the final state.
 *   q, k [B,H,T,DK] dtype; v [B,H,T,DV] dtype; beta, g [B,H,T] fp32 (g = per-token log decay,
 *   summed within each chunk of C tokens by the kernel); h0 [B,H,DK,DV] fp32 or NULL (zero);
 *   o [B,H,T,DV] fp32 (scaled by `scale`); h_final [B,H,DK,DV] fp32 or NULL.
 *   Supported: C = 64 or 128, DK = DV = 128, T % C == 0, T <= 4 194 304 (per-chain addressing is
 *   32-bit; a longer sequence is PF_ERR_ARG).  The kernels run 64-token chunks; C = 128
 *   (the reference's chunk) is served by them over T / 64 chunks — the chunked forward's result
 *   does not depend on the chunk size, only the blocking of its arithmetic does.
 * ------------------------------------------------------------------------------------------ */
size_t pf_gdn_workspace_bytes(int B, int H, int T, int C, int DK, int DV, int dtype);
void* pf_gdn_setup(int B, int H, int T, int C, int DK, int DV, int dtype);
/* The same workspace in two steps, for a registry whose setup takes no arguments (the
 * reference's FusedKernel calls setup_sym() bare, fused.py:102-107): pf_gdn_create returns an
 * empty handle (allocates nothing); pf_gdn_reserve grows it to the shape's size (PF_OK, PF_ERR_ARG
 * for an unsupported shape, PF_ERR_ALLOC).  A reserve that does not grow allocates nothing and is
 * safe under HIP graph capture; one that grows waits for the device and must run outside it.
 * Growing frees the old buffer: a HIP graph captured on the handle before a growth still
 * addresses it and must be captured again.  The fp32 layout of a shape holds its bf16 layout, so
 * a handle reserved for the fp32 size serves both dtypes of that shape without growing.
 * pf_gdn_setup(shape) == pf_gdn_create() + pf_gdn_reserve(shape); pf_gdn_teardown frees either. */
void* pf_gdn_create(void);
int pf_gdn_reserve(void* ws, int B, int H, int T, int C, int DK, int DV, int dtype);
int pf_gdn_exec(const void* q, const void* k, const void* v, const float* beta, const float* g,
                const float* h0, float* o, float* h_final, int B, int H, int T, int C, int DK,
                int DV, int dtype, float scale, void* ws, void* stream);
void pf_gdn_teardown(void* ws);

/* The same forward with no workspace argument and no allocation of any kind: no counterpart in
 * the reference.  It is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).  Its workspace is a
 * file-scope device array of 40 MiB (bf16: up to 4 964 chunks of 64 tokens, the B4 H16 T4096
 * headline included; fp32: up to 1 270); a larger input returns PF_ERR_SCRATCH and launches
 * nothing.  The array's device address is looked up once per device on the first call there
 * (make that call outside any graph capture).  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (different streams, or threads) race; serialise them.  Same
 * arguments as pf_gdn_exec otherwise. */
int pf_gdn_exec_static(const void* q, const void* k, const void* v, const float* beta,
                       const float* g, const float* h0, float* o, float* h_final, int B, int H,
                       int T, int C, int DK, int DV, int dtype, float scale, void* stream);

/* The two stages pf_gdn_exec enqueues, exposed so a caller can time or overlap them
 * separately.  Stage 1 (chunk-local, one workgroup per chunk) writes the within-chunk gate
 * cumsum G and T = (I + A)^-1 into the workspace, and records `scale` there — the work of the
 * reference's kkt_gated_native_v2 + tri_inv_rec_unroll nodes (fused.py:482-517,
 * registry.py:107-127); for fp32 operands it also writes the gated causal score P (multiplied by
 * `scale`, the reference's gated_qk node), which the bf16 stage 2 forms itself from the q and k
 * rows it stages (q is then not read by stage 1).  Stage 2 (scan + output, state
 * register-resident) reads them, the scale included, and writes o and h_final — the reference's
 * WY einsums, chunk_h_scan and qkv_flash_native_v2 (_gdn_full.py:199-233, scan_lib.cpp:81-99,
 * qkv_fused_lib.cpp:148-165).  Stage 2 must be ordered after stage 1 on the same workspace (same
 * stream, or an event). */
int pf_gdn_chunk_local_exec(const void* q, const void* k, const float* beta, const float* g,
                            int B, int H, int T, int C, int DK, int DV, int dtype, float scale,
                            void* ws, void* stream);
int pf_gdn_scan_output_exec(const void* q, const void* k, const void* v, const float* beta,
                            const float* h0, float* o, float* h_final, int B, int H, int T, int C,
                            int DK, int DV, int dtype, void* ws, void* stream);

/* ------------------------------------------------------------------------------------------
 * Fused KDA forward (per-channel decay).  Replaces the lowered KDA program of
 * examples/attention/_kda_full.py (host gate prep :78-103, the gated kkt / per-dim flash
 * templates template.py:335-397 and the per-dim chunk_h_scan of transforms/kda.py:20-85 with
 * scan_fused.h:143-180), the per-channel gate being applied on the device: stage 1 forms the
 * gated operands k e^G, k e^-G and q e^G from g, inverts (I + A) and builds the WY factor W and
 * T diag(beta) (fp32 operands: also k e^{G_last - G}, U and the causal score); with bf16 operands
 * stage 2 forms U = T diag(beta) v and the causal score from the tiles it stages, and it carries
 * the state in registers with a per-channel decay.
 * Math: kda_reference (_kda_full.py:42-76) plus an initial state h0 and the final state.
 *   q, k [B,H,T,DK] and v [B,H,T,DV] of `dtype`; beta [B,H,T] fp32; g [B,H,T,DK] fp32
 *   (per-token, per-channel log decay, summed within each chunk of C tokens by the kernel);
 *   h0 [B,H,DK,DV] fp32 or NULL; o [B,H,T,DV] fp32 (scaled by `scale`); h_final [B,H,DK,DV]
 *   fp32 or NULL.  Supported: dtype PF_DTYPE_BF16 (bf16 MFMA) or PF_DTYPE_F32 (fp32
 *   operands and fp32 MFMA throughout), C = 64 or 128 (run as 64-token chunks),
 *   DK = DV = 128, T % C == 0, T <= 4 194 304.  The workspace holds the stage-1 images in the
 *   operand type.
 * ------------------------------------------------------------------------------------------ */
size_t pf_kda_workspace_bytes(int B, int H, int T, int C, int DK, int DV, int dtype);
void* pf_kda_setup(int B, int H, int T, int C, int DK, int DV, int dtype);
/* Two-step form of pf_kda_setup, as pf_gdn_create / pf_gdn_reserve above. */
void* pf_kda_create(void);
int pf_kda_reserve(void* ws, int B, int H, int T, int C, int DK, int DV, int dtype);
int pf_kda_exec(const void* q, const void* k, const void* v, const float* beta, const float* g,
                const float* h0, float* o, float* h_final, int B, int H, int T, int C, int DK,
                int DV, int dtype, float scale, void* ws, void* stream);
void pf_kda_teardown(void* ws);

/* ------------------------------------------------------------------------------------------
 * Standalone kkt + triangular inverse over M independent chunks.
 * Replaces the kkt_gated_native FusedNode (fused.py:482-499, kkt_fused_lib.cpp:98-113)
 * followed by tri_inv_rec_unroll (registry.py:107-127):
 *   A = strictly_lower(beta_i * safe_exp(G_i - G_j) * k_i.k_j), T = (I + A)^-1
 *   k [M*C, DK] dtype; g, beta [M*C] fp32 (g_is_cumsum = 1: g already holds G);
 *   A_out [M,C,C] fp32 or NULL; T_out [M,C,C] fp32.  Supported: C = 64, DK = 128.
 * ------------------------------------------------------------------------------------------ */
int pf_kkt_inv_exec(const void* k, const float* g, const float* beta, float* A_out, float* T_out,
                    int M, int C, int DK, int dtype, int g_is_cumsum, void* stream);

/* ------------------------------------------------------------------------------------------
 * Opaque unit-lower triangular inverse.  Replaces the pto-kernels tri_inv call of
 * registry.py:124 (`tri_inv(out, A_upper, mi, C, M, 0, cu_seqlens=None, block_dim)`), which
 * inverts strictly-upper fp16 input: this one takes the strictly-LOWER fp32 A directly.
 *   A [M,C,C] fp32 (only the strictly-lower part is read); T_out [M,C,C] fp32 = (I + A)^-1.
 *   Supported: C in {16, 32, 48, 64, 128} (the reference contract is {16, 32, 64, 128}).
 * ------------------------------------------------------------------------------------------ */
int pf_tri_inv_exec(const float* A, float* T_out, int M, int C, void* stream);

/* ------------------------------------------------------------------------------------------
 * Stage kernels of the compile stack's fused nodes.  They keep no state between calls, so their
 * setup functions return NULL and their teardowns accept it; they exist so that a recipe of the
 * reference's shape (fused.py:119-127: setup_sym / teardown_sym around a persistent runner,
 * fused.py:93-115) binds them unchanged.  Replace scan_setup / scan_teardown
 * (scan_lib.cpp:81-88, :99), kkt_setup / kkt_setup_v2 / kkt_teardown
 * (kkt_fused_lib.cpp:98-104, :115, :119-126) and qkv_setup / qkv_setup_v2 / qkv_teardown
 * (qkv_fused_lib.cpp:123-130, :143, :147-155).  Supported (C, D): C in {16, 32, 64, 128} (bf16
 * needs C >= 32), D in {64, 128}.
 *
 * Row addressing shared by the gated-qk stage: chunk m = c*H + h of an [nc*C, H, D] token
 * layout holds rows (c*C + i)*H + h, i < C.  H = 1 is the native [M, C, D] batch (M = nc).
 * ------------------------------------------------------------------------------------------ */

/* Gated a bᵀ:  L[m,i,j] = (a'_i · b'_j) · exp(min(g_i + log beta_i − g_j, 0)) · mask_ij
 *   a' = a ⊙ a_scale, b' = b ⊙ b_scale when the scales are given (fp32, same addressing as a/b).
 *   Replaces kkt_exec / kkt_exec_v2 (kkt_fused_lib.cpp:105-135; recipes kkt_gated, gated_qk and
 *   their _native / _native_v2 forms, fused.py:200-290) and, with scales and g = beta = NULL,
 *   pro_exec / pro_exec_v2 (prologue_fused_lib.cpp; recipes qk_prologue*, fused.py:293-340).
 *   a, b: dtype, rows of D; g, beta: fp32 [nc*C, H] or NULL (0 / 1); mask: [C,C] fp32 or NULL
 *   (then causal = 1 keeps i >= j, 0 keeps i > j); L: [nc*C, H, C] in out_dtype (fp32 or bf16). */
void* pf_gated_qk_setup(void);
void pf_gated_qk_teardown(void* ws);
int pf_gated_qk_exec(const void* a, const void* b, const float* a_scale, const float* b_scale,
                     const float* g, const float* beta, const float* mask, void* L, int nc, int H,
                     int C, int D, int dtype, int causal, int out_dtype, void* stream);

/* chunk_o flash: o[m] = causal_incl( (q'kᵀ') · exp(min(g_i + log beta_i − g_j, 0)) ) · v[m], the
 * score never leaving the chip.  q' = q ⊙ q_scale, k' = k ⊙ k_scale when given (per-channel gate,
 * the qkvp form).  Replaces qkv_exec / qkv_exec_v2 (qkv_fused_lib.cpp:123-165; recipes
 * qkv_flash_native*, fused.py:353-395) and qkvp_exec* (qkv_prologue_fused_lib.cpp; recipes
 * qkvp_flash_native*, fused.py:411-444).  q, k, v [M,C,D] dtype; scales [M,C,D] fp32 or NULL;
 * g, beta [M,C] fp32 or NULL; o [M,C,D] fp32. */
void* pf_qkv_flash_setup(void);
void pf_qkv_flash_teardown(void* ws);
int pf_qkv_flash_exec(const void* q, const void* k, const void* v, const float* q_scale,
                      const float* k_scale, const float* g, const float* beta, float* o, int M,
                      int C, int D, int dtype, void* stream);

/* Resident-state chunk recurrence (chunk_h_scan).  Per (b,h), chunk c:
 *   h_out[b,c,h] = S;   S = decay[b,h,c] ⊙ S + k_cᵀ (u_c − w_c S)
 * decay is a scalar per chunk ([B,H,nc], perdim = 0) or scales state row d ([B,H,nc,D],
 * perdim = 1).  Replaces scan_exec (scan_lib.cpp:81-99, scan_fused.h:198-262; per-dim form
 * :143-180; recipe chunk_h_scan, fused.py:168-182), which is fixed to C = D = 128 and starts from
 * zero: here h0 [B,H,D,D] fp32 (or NULL = zero) is accepted.  w, u, k [B,nc,C,H,D] dtype;
 * h_out [B,nc,H,D,D] in out_dtype; final_state [B,H,D,D] fp32 or NULL. */
void* pf_scan_setup(void);
void pf_scan_teardown(void* ws);
int pf_scan_exec(const void* w, const void* u, const void* k, const float* decay,
                 const float* h0, void* h_out, float* final_state, int B, int H, int nc, int C,
                 int D, int dtype, int perdim, int out_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PTO_FUSER_HIP_H */
