/* catfuse_amd — C-ABI of the gfx950 HIP kernels behind the CATFuse-SF
 * spatio-temporal fused SNN inference path.
 *
 * Conventions for every entry point:
 *   - device pointers are raw HIP device addresses; "nullable" pointers may
 *     be NULL;
 *   - sizes are int64, LIF parameters are passed as the SpikingJelly-level
 *     doubles (rounded to fp32 inside exactly as torch rounds a Python float
 *     against an fp32 tensor);
 *   - `stream` is a hipStream_t; every call is asynchronous on it, never
 *     allocates, never synchronises;
 *   - the return value is a hipError_t (0 = success; hipErrorInvalidValue
 *     for rejected arguments, checked on the host before any launch).
 * Tensor layouts: "NCHW" = [T][B][C][H][W] fp32 boundary tensors (the
 * layout SpikingJelly multi-step modules exchange); "NHWC16" = fp16
 * [images][H][W][Cp] staging of conv inputs.
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the hpcyhr/CATFuse source tree).
 */
#ifndef CATFUSE_AMD_H
#define CATFUSE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Route words written by cf_route_from_nnz. */
#define CF_ROUTE_ZERO 0   /* StaticZero: count_nonzero(x) == 0          */
#define CF_ROUTE_SPARSE 1 /* SparseFlow: 1 - nnz/numel > threshold      */
#define CF_ROUTE_DENSE 2  /* DenseKeep                                  */

/* Count blocks: CF_COUNT_BLOCK_WORDS uint64 in device memory, [0] the
 * accumulator of a producer pass (zero between passes), [1] the count the
 * last completed pass published, [16*(g+1)] for g < 16 the accumulators of
 * the pass's workgroup groups (zero between passes).  Producer passes
 * (cf_pack_input, cf_scan_nhwc, and cf_conv_mfma / cf_conv_halo through
 * nz_out) add into their group word with one atomic per workgroup; the
 * workgroup completing a group adds the group total to [0], and the one
 * completing [0] stores the pass total in [1]; each clears what it completed.
 * The owner zeroes a block once; passes publishing into one block must not
 * overlap (stream order).  Readers (the routing of cf_conv_mfma /
 * cf_conv_halo, cf_route_from_nnz) read [1] in later launches.  Replaces the
 * host-side count_nonzero(x).item() of
 * catfuse/sparseflow/ops/st_fusion_conv_bn_lif.py:512-514. */
#define CF_COUNT_BLOCK_WORDS 272

/* Status bits OR-ed into the device status word by cf_pack_input. */
#define CF_STATUS_INEXACT_FP16 1u

int cf_version(void);
const char* cf_error_string(int code);

/* Multi-step LIF over T steps with the membrane potential kept on chip.
 * Replaces catfuse/sparseflow/lif_seq_kernel.py:51-90 lif_sequential
 * (mode 0), catfuse/kernels/partial_fusion_conv_bn_lif_impl.py:157-189
 * _launch_bn_lif_state_carry (mode 1),
 * catfuse/kernels/partial_fusion_conv_bn_add_lif_impl.py:125-158 (mode 2),
 * catfuse/kernels/add_lif.py:112-151 triton_add_lif_blocked (mode 3),
 * benchmarks/add_bn_lif_min.py:131-226 run_fusion (mode 4).
 *   input current per step and neuron n (channel c = (n / HW) % C):
 *     0: z          1: z*scale[c] + shift[c]       2: (z*scale[c] + shift[c]) + z2
 *     3: z + z2     4: (z + z2)*scale[c] + shift[c]
 *   z, z2: [T][N] fp32; v_in, v_out: [N] fp32 (nullable; NULL v_in starts at
 *   v_reset for hard reset, 0 for soft); spike: [T][N] fp32 (spike_dtype 0)
 *   or uint8 (spike_dtype 1).  hard_reset = 0 means soft reset (v_reset
 *   None in SpikingJelly). */
int cf_lif_multistep(const float* z, const float* z2, const float* scale, const float* shift,
                     int mode, const float* v_in, void* spike, int spike_dtype, float* v_out,
                     int64_t T, int64_t N, int64_t C, int64_t HW, double tau, double v_th,
                     double v_reset, int hard_reset, int decay_input, void* stream);

/* AvgPool2d(2,2) -> LIF over T steps.  Replaces
 * catfuse/kernels/avgpool_lif.py:61-190 (avgpool_lif_block_kernel /
 * triton_avgpool_lif_blocked).  x: [T][NC][H][W]; spike: [T][NC][H/2][W/2];
 * v_in/v_out: [NC][H/2][W/2] (nullable). */
int cf_avgpool2x2_lif(const float* x, const float* v_in, void* spike, int spike_dtype,
                      float* v_out, int64_t T, int64_t NC, int64_t H, int64_t W, double tau,
                      double v_th, double v_reset, int hard_reset, int decay_input, void* stream);

/* One pass over a conv input x [NB][C][H][W] fp32: fp16 NHWC staging
 * (xp: [NB][H][W][Cp], Cp % 32 == 0, nullable), per-pixel channel-group
 * activity bits (act: uint32 [NB][H][W], bit g <=> some |x| > threshold in
 * channels [g*group_size, (g+1)*group_size), nullable), nonzero count
 * (count_nonzero(x) published in the count block nnz, nullable; see
 * "Count blocks" below) and exactness status (nullable).
 * Replaces the channel half of catfuse/sparseflow/prescan.py:32-54,153-189
 * and the count_nonzero of
 * catfuse/sparseflow/ops/st_fusion_conv_bn_lif.py:512-514. */
int cf_pack_input(const float* x, int64_t NB, int64_t C, int64_t H, int64_t W, int64_t Cp,
                  void* xp, uint32_t* act, int group_size, float threshold,
                  unsigned long long* nnz, uint32_t* status, void* stream);

/* Activity bits and nonzero count of cf_pack_input (same definitions, same
 * act layout) from an fp16 NHWC tensor xp [NB][H][W][Cp] that a fused conv
 * wrote as its output copy (channels >= C zero), for a SparseFlow layer whose
 * input carries one: no fp32 pass.  group_size must be a multiple of 8.
 * Replaces, like cf_pack_input, the channel reduction of
 * catfuse/sparseflow/prescan.py:32-45,184 and the count of
 * catfuse/sparseflow/ops/st_fusion_conv_bn_lif.py:510-524. */
int cf_scan_nhwc(const void* xp, int64_t NB, int64_t H, int64_t W, int64_t Cp, int64_t C,
                 uint32_t* act, int group_size, float threshold, unsigned long long* nnz,
                 void* stream);

/* fp16 NHWC xp [NB][H][W][cp] -> fp32 NCHW out [NB][C][H][W]: the fp32 form
 * of a fused conv output kept only as its NHWC copy, produced when a module
 * outside the fused chain first reads it.  No counterpart in the reference
 * (whose fused layers always write fp32 spikes, e.g.
 * catfuse/implementations/sparse_flow.py:236-238). */
int cf_nhwc_to_nchw(const void* xp, float* out, int64_t NB, int64_t C, int64_t H, int64_t W,
                    int64_t cp, void* stream);

/* Global average pool of an fp16 NHWC copy xp [NB][HW][cp] (channels >= C
 * zero): out [NB][C] fp32 = (sum over the HW pixels) * float(1)/HW, which is
 * torch's GPU mean (AdaptiveAvgPool2d((1, 1)) = mean over H, W) bit for bit
 * for the integer values a fused conv's copy holds.  No counterpart in the
 * reference (the network head after the fused layers is SpikingJelly's
 * layer.AdaptiveAvgPool2d); it reads the copy instead of materialising the
 * fp32 feature map.  desc (nullable): the copy's output descriptor (see
 * cf_conv_mfma): an all-zero copy pools to zeros, an aliased one is read
 * where it points. */
int cf_global_avgpool_nhwc(const void* xp, const void* desc, float* out, int64_t NB, int64_t HW,
                           int64_t C, int64_t cp, void* stream);

/* Output descriptors.  A fused conv given an output descriptor (16 bytes of
 * device memory: uint32 copy, uint32 vstate, pointer alias) records there
 * how it left its outputs: copy 0 written, 1 all zero and the fp16 copy not
 * written, 2 equal to the copy at alias (its identity) and not written;
 * vstate 1: every pixel of channel c holds v_chan[c] and v_out was not
 * written.  cf_resolve_copy makes the buffer xp (bytes, a multiple of 16,
 * 16-byte aligned) hold the values when it was not written (zeros, or the
 * aliased bytes); cf_expand_state fills v [B][C][HW] from v_chan when
 * vstate is 1.  Both leave written outputs alone.  No counterpart in the
 * reference (its fused layers always write their outputs). */
int cf_resolve_copy(void* xp, int64_t bytes, const void* desc, void* stream);
int cf_expand_state(float* v, const float* v_chan, const void* desc, int64_t B, int64_t C,
                    int64_t HW, void* stream);

/* Token-major fp32 x [rows][C] (a transformer's [T, B, N, C] activations)
 * -> its fp16 copy xp [rows][cp] (cp >= C, cp % 8 == 0, channels >= C zero),
 * count_nonzero(x) published in the count block nnz (nullable) and the
 * exactness status (nullable): the staging of a fused Linear's input, read
 * by cf_conv_mfma as an NHWC image of the N tokens.  Replaces the fp32 input
 * of the Linear layers of models/spikformer_github.py:77-92,126-137 (the
 * reference leaves Linear -> BN1d -> LIF unfused, substitute.py:559-567). */
int cf_pack_tokens(const float* x, int64_t rows, int64_t C, int64_t cp, void* xp,
                   unsigned long long* nnz, uint32_t* status, void* stream);

/* fp16 token copy xp [rows][cp] -> fp32 out [rows][C]: the fp32 form of a
 * fused token layer's output kept only as its copy.  No counterpart. */
int cf_tokens_to_f32(const void* xp, float* out, int64_t rows, int64_t C, int64_t cp,
                     void* stream);

/* Spikformer spiking self-attention core + its LIF over T, on the matrix
 * cores: per (t, b, head) z = ((Q K^T) V) * scale with binary Q, K, V of
 * N tokens x head_dim (= 32) channels, evaluated exactly as Q (K^T V) in
 * integers and rounded once by the scale; then LIF_T(z) -> spikes.  Q, K, V
 * are fp16 token copies [T*B][N][pitch] with head h at channel
 * off + 32h (off = qoff / koff / voff; q, k, v may be one concatenated QKV
 * tensor); out fp16 [T*B][N][cp_out] (head h at channel 32h); v_in / v_out
 * fp32 [B][N][heads*32] (nullable); nnz (nullable): count block of the Q, K,
 * V tensor (one concatenated tensor): a published count of zero takes the
 * zero route (no operand reads, no MFMAs, z = 0); nz_out (nullable): count
 * block of the output (workgroups with a spike).  out_desc (nullable): the
 * output's descriptor (see cf_conv_mfma), with zero_info the caller's
 * knowledge of the LIF on z = 0 (cf_bias_response of a zero affine: bit 0,
 * it never fires over T; bit 1, the caller holds its final potential, the
 * same for every neuron): on the zero route from the initial state with
 * bit 0 the launch stores no spikes (copy recorded all zero), and with bit
 * 1 no state either (vstate 1).  N <= 256.  Replaces the SSA core of
 * models/spikformer_github.py:139-160 (q @ k^T * scale, @ v, attn_lif) and
 * the reference's spike-matmul kernels (sparseflow/sparse_bmm_kernel.py:40-358,
 * sparse_attention_kernel.py:24-118). */
int cf_spike_attention_lif(const void* q, const void* k, const void* v, int64_t qoff,
                           int64_t koff, int64_t voff, int64_t pitch, void* out, int64_t cp_out,
                           const float* v_in, float* v_out, const unsigned long long* nnz,
                           unsigned long long* nz_out, void* out_desc, int zero_info,
                           int64_t T, int64_t B, int64_t N, int64_t heads, int64_t head_dim,
                           double scale, double tau, double v_th, double v_reset, int hard_reset,
                           int decay_input, void* stream);

/* The same core for any token count (N < 65536, head_dim * N < 2^24) and
 * head_dim 32 or 64, in two launches: K^T V of every (t, b, head) reduced
 * over all N tokens into the caller's workspace kv_ws (fp32
 * [T*B*heads][head_dim][head_dim], exact integers), then per (b, head,
 * 128-token block) Y = Q (K^T V) on the matrix cores with K^T V as two exact
 * fp16 limbs, z = Y * scale (one rounding), the LIF over T.  Same values as
 * cf_spike_attention_lif where both apply (the exact Y, the same rounding);
 * other arguments, layouts (head h at channels off + h*head_dim), routes
 * and descriptors as cf_spike_attention_lif.  Replaces the same reference
 * interfaces, for the shapes of models/spikformer_github.py:332-350
 * (head_dim 64) and its two-pool patch splitter (:240-242, 3,136 tokens at
 * 224 x 224). */
int cf_spike_attention_kv_lif(const void* q, const void* k, const void* v, int64_t qoff,
                              int64_t koff, int64_t voff, int64_t pitch, void* out,
                              int64_t cp_out, const float* v_in, float* v_out, float* kv_ws,
                              const unsigned long long* nnz, unsigned long long* nz_out,
                              void* out_desc, int zero_info, int64_t T, int64_t B, int64_t N,
                              int64_t heads, int64_t head_dim, double scale, double tau,
                              double v_th, double v_reset, int hard_reset, int decay_input,
                              void* stream);

/* A plain Linear (no neuron) over a token-major fused output kept as its
 * fp16 copy xp [M][cp] (cp >= K; a fused Linear-LIF's output, read through
 * its output descriptor desc, nullable): out [M][O] fp32 = x w^T + bias
 * (w [O][K] fp32, bias [O] nullable; O <= 4096), accumulated in fp32 in a
 * fixed order (deterministic; not torch's order, so equal to torch's
 * F.linear within fp32 rounding).  For a network's last classifier layer
 * after fused Linear-LIF layers, which otherwise needs the fp32 form of its
 * input first.  No counterpart in the reference (nn.Linear there). */
int cf_linear_tokens(const void* xp, const void* desc, const float* w, const float* bias,
                     float* out, int64_t M, int64_t K, int64_t cp, int64_t O, void* stream);

/* MaxPool2d(kernel_size, stride, padding) of an fp16 NHWC copy xp
 * [NB][H][W][cp] -> out [NB][Ho][Wo][cp] (padded positions ignored, as
 * torch's max_pool2d; 2*padding <= kernel_size so every window has an input);
 * nz_out (nullable) receives the output's count block.  Exact for spikes.
 * in_desc (nullable): the input copy's output descriptor (read where its
 * producer left the values); out_desc (nullable) receives the output's: an
 * all-zero input (in_desc ZERO) with out_desc given writes no output, only
 * the descriptor (all zero) and a zero count.  Replaces the MaxPool2d
 * between fused Conv-BN-LIF stages of models/spikformer_github.py:181-254
 * (SPS), which the reference runs in torch on the fp32 spikes. */
int cf_maxpool_nhwc(const void* xp, const void* in_desc, void* out, void* out_desc, int64_t NB,
                    int64_t H, int64_t W, int64_t cp, int64_t kernel_size, int64_t stride,
                    int64_t padding, unsigned long long* nz_out, void* stream);

/* route = ZERO if the count block's published count k (nnz[1]) is 0, SPARSE
 * if 1 - k/numel > sparse_threshold (in double), else DENSE.  Replaces the host decision at
 * catfuse/sparseflow/ops/st_fusion_conv_bn_lif.py:510-524. */
int cf_route_from_nnz(const unsigned long long* nnz, int64_t numel, double sparse_threshold,
                      int32_t* route, void* stream);

/* *p = 0 by a one-thread kernel (graph-capture safe). */
int cf_zero_counter(unsigned long long* p, void* stream);

/* Prescan tile reduction: ag_mask / tile_class int32 [NB*GH*GW] from the
 * activity bits of cf_pack_input, GH = ceil(Ho/block_h), GW =
 * ceil(Wo/block_w).  Replaces catfuse/sparseflow/fast_prescan_v2.py:92-137
 * fast_spike_prescan_2d_v2 and prescan.py:153-189 _prescan_2d_impl
 * (bit-exact contract: same masks and classes). */
int cf_prescan_tiles(const uint32_t* act, int64_t NB, int64_t H, int64_t W, int64_t Ho,
                     int64_t Wo, int64_t kernel_size, int64_t stride, int64_t padding,
                     int64_t block_h, int64_t block_w, int64_t num_groups, int32_t* ag_mask,
                     int32_t* tile_class, void* stream);

/* Active-tile compaction and dispatch score on the device: from ag_mask
 * [T][ntiles] (cf_prescan_tiles, ntiles = B*GH*GW, num_groups groups),
 * order[0] = the number of tiles active at some step (any bit of
 * ag_mask[t][tile] set for some t < T), order[1 ..] = the tile indices,
 * active tiles first, each part ascending.  With tau >= 0 the launch also
 * scores the layer as the reference's execution-grounded dispatch does,
 * over the tile's time steps (the conv skips a group only where it is
 * silent at all of them): R = 1 - (set bits of the OR over t of
 * ag_mask[t][tile]) / (ntiles * num_groups), S = R * macs_per_tile (dense
 * MACs per image / tiles per image); unless R >= 0.99,
 * or R >= r_min and S > tau, order[0] is -1 and cf_conv_mfma then takes the
 * dense route (same results).  tau < 0: no score.  order holds 1 + ntiles
 * int32; ntiles < 2^30.  One workgroup, no host synchronisation, graph-
 * capture safe.  Replaces the host-synchronising
 * catfuse/sparseflow/sparse_conv2d_kernel.py:113-123 _build_active_tile_ids
 * (torch.nonzero over tile_class != TILE_ZERO) feeding the active-tile
 * launch at :1102-1163, and the host-side decision of
 * catfuse/sparseflow/dispatch.py:860-1000 (make_dispatch_decision, R_l,
 * S_l, tau, R_min); here every tile keeps its workgroup (inactive ones run
 * the LIF epilogue on the bias drive) and the order makes the active ones
 * run first (cf_conv_mfma tile_order). */
int cf_compact_tiles(const int32_t* ag_mask, int64_t T, int64_t ntiles, int64_t num_groups,
                     double macs_per_tile, double tau, double r_min, int32_t* order,
                     void* stream);

/* Conv weight staging for cf_conv_mfma: fp32 w [Cout][Cin][KH][KW] ->
 * fp16 hi/lo limbs with a per-channel power-of-two prescale (2*Coutp*KH*KW*Cp
 * halves, fragment-major: per limb, 32-channel tile, tap and 16-channel K
 * step one 64-lane x 8-half MFMA A fragment), plus the folded epilogue affine alpha/beta [Coutp]
 * (alpha = bn_scale / prescale, beta = bn_shift + bias*bn_scale; bn_* and
 * bias nullable).  With w_packed == NULL only alpha/beta are written (no
 * prescale), the form cf_conv_direct consumes.  Replaces the weight caches
 * of catfuse/implementations/dense_keep.py:73-95 (_ensure_fold) and
 * catfuse/implementations/sparse_flow.py:92-99 (_ensure_w_cl). */
int cf_pack_conv_weights(const float* w, int64_t Cout, int64_t Cin, int64_t KH, int64_t KW,
                         int64_t Coutp, int64_t Cp, const float* bn_scale, const float* bn_shift,
                         const float* bias, void* w_packed, float* alpha, float* beta,
                         void* stream);

/* Fused Conv -> BN -> LIF (epilogue 0), Conv -> BN -> z (epilogue 1) or
 * Conv -> BN -> AvgPool2d(2, 2) -> LIF (epilogue 2) on the matrix cores, all
 * T steps in one launch.
 *   x: NHWC16 [T*x_img_tstride + B][H][W][Cp] from cf_pack_input;
 *   out: NCHW [T][B][Cout][Ho][Wo] spikes or z;
 *   out_nhwc (nullable): the same values as fp16 NHWC [T*B][Ho][Wo][cp_out]
 *   (Cout <= cp_out <= Coutp, channels >= Cout zero) — the staging layout
 *   the next fused conv reads, so it needs no separate pack pass;
 *   identity (nullable, NCHW like out): identity_mode 1 adds it to the
 *   spikes (SEW ADD, catfuse/patterns.py:672-737), identity_mode 2 adds it
 *   to z before the LIF (BN -> Add -> LIF,
 *   catfuse/kernels/partial_fusion_conv_bn_add_lif_impl.py:76-123);
 *   identity_nhwc (nullable, mode 1 only): the same identity as fp16 NHWC
 *   [T*B][Ho][Wo][cp_id] (cp_id >= Cout, a multiple of 4), read instead of
 *   the NCHW one (exact for the integer values a SEW ADD identity holds);
 *   v_in/v_out: [B][Cout][Ho][Wo] (nullable, except that layers taking the
 *   halo kernel (cf_conv_halo) need v_out for the LIF epilogue when T > 2:
 *   the state passes between its time blocks through it);
 *   tile_h/tile_w > 0 selects rectangular pixel tiles aligned with the
 *   prescan tiles (tile_h*tile_w in {64,128}) and enables SparseFlow chunk
 *   skipping from ag_mask ([T][B*GH*GW]) when nnz is non-NULL; tile_h = 0
 *   selects flat pixel tiles (dense).  With prescan groups narrower than 32
 *   channels, a silent 16-channel half of a chunk also skips its MFMAs.
 *   tile_order (nullable, needs ag_mask; [1 + B*GH*GW] as cf_compact_tiles
 *   writes it): on the SparseFlow route the halo kernel gives each XCD an
 *   equal share of the tiles active at some step, dispatched before the
 *   inactive ones (which only run the epilogue), and takes the dense route
 *   instead when tile_order[0] < 0 (the dispatch score rejected SparseFlow);
 *   ignored by the flat-tile kernel and by the other routes.  nnz (nullable, read only) is the
 *   count block of the input: its published count k (exact, from
 *   cf_pack_input / cf_scan_nhwc, or the producing conv's nz_out) routes
 *   the launch: k == 0 StaticZero (no K loop), SparseFlow when ag_mask is
 *   given and 1 - k/numel > sparse_threshold, dense otherwise.  numel is the
 *   input's element count T*B*Cin*H*W; the halo kernel takes its real
 *   channel count Cin = numel/(T*B*H*W) (when that divides and is at most
 *   Cp) and skips the products of zero-padded 16-channel input halves, and
 *   of output waves whose 32 channels all lie beyond Cout (exact zeros or
 *   discarded outputs: the results are those of the full evaluation).  nz_out
 *   (nullable) is the count block the launch publishes for its output: the
 *   number of workgroups that stored a nonzero value (0 iff the output is
 *   all zero), so the next fused conv can route on it without a counting
 *   pass.  All routes give bit-identical results.
 *   Output descriptors (each nullable, see cf_resolve_copy): x_desc /
 *   id_desc are those of the input's / identity's copies as their producers
 *   left them: an all-zero input takes StaticZero without reading x, an
 *   all-zero identity is read as zeros, aliased ones where they point.
 *   out_desc receives this launch's.  bias_info (needs out_desc) is what
 *   the caller knows from cf_bias_response for this layer and T: bit 0, no
 *   channel fires on its bias drive alone; bit 1, the caller holds the
 *   per-channel final potentials.  A halo launch on StaticZero with the
 *   lean epilogue (out_nhwc only), no v_in and bit 0 writes no out_nhwc and
 *   records it as all zero (no identity, or an all-zero one; nz_out
 *   publishes 0) or as an alias of the identity's copy (id_desc given, the
 *   identity a fused layer's copy of spike counts, and cp_id == cp_out;
 *   nz_out publishes nonzero unless id_nnz, the identity's count block,
 *   says zero); with bit 1 such a launch also leaves v_out unwritten
 *   (vstate 1: every pixel of channel c holds v_final[c]).  Every other
 *   launch writes its outputs and records so.  A caller that passes
 *   out_desc reads the outputs through it (or hands it on as x_desc /
 *   id_desc).
 *   Epilogue 2 (stride-1 3x3 convs on 8x8 tiles, the halo kernel): each 2x2
 *   window of BN outputs is summed as ((z00 + z01) + z10) + z11, times
 *   0.25 (the order of cf_avgpool2x2_lif, so the spikes equal epilogue 1
 *   followed by cf_avgpool2x2_lif bit for bit), and drives the pooled
 *   neuron's LIF; out_nhwc (required, out must be NULL) then holds the
 *   pooled spikes [T*B][Ho/2][Wo/2][cp_out] (cp_out a multiple of 4),
 *   v_in/v_out the pooled state [B][Cout][Ho/2][Wo/2]; Cout a multiple of
 *   32, no identity; bias_info from cf_bias_response with pool = 1 (a
 *   StaticZero launch with no v_in and bit 0 writes no copy, records it as
 *   all zero, and with bit 1 leaves v_out to the per-channel potentials;
 *   every other pooled launch writes its outputs) (reference: the F8 chain of
 *   catfuse/kernels/conv_pool_lif.py:94-178, whose z makes a round trip
 *   through HBM).
 * Replaces catfuse/implementations/dense_keep.py:97-155 (DenseKeep.forward),
 * catfuse/implementations/sparse_flow.py:186-270 (SparseFlow.forward ->
 * catfuse/sparseflow/streamfuse_kernel.py:32-187), and
 * catfuse/sparseflow/fused_conv_bn_lif_kernel.py:342-539. */
int cf_conv_mfma(const void* x, const void* w_packed, const float* alpha, const float* beta,
                 const float* v_in, float* v_out, float* out, void* out_nhwc, int64_t cp_out,
                 const float* identity, const void* identity_nhwc, int64_t cp_id,
                 int identity_mode, const int32_t* ag_mask, const int32_t* tile_order,
                 const unsigned long long* nnz, unsigned long long* nz_out,
                 const void* x_desc, const void* id_desc, void* out_desc, int bias_info,
                 const unsigned long long* id_nnz, int64_t numel, double sparse_threshold,
                 int64_t T,
                 int64_t B, int64_t Cp, int64_t Cout, int64_t Coutp, int64_t H, int64_t W, int64_t Ho, int64_t Wo, int64_t KH,
                 int64_t KW, int64_t stride, int64_t pad, int64_t x_img_tstride, int64_t tile_h,
                 int64_t tile_w, int64_t group_size, int epilogue, double tau, double v_th,
                 double v_reset, int hard_reset, int decay_input, void* stream);

/* 3x3 or 1x1 Conv (stride 1 or 2) -> BN -> LIF / z with the input halo of each
 * (tile_h x tile_w) output tile staged in LDS once per 32-channel chunk and
 * up to 4 time steps accumulated per tile (weights fetched once per tap for
 * all of them).  cf_conv_mfma forwards every 3x3 layer and every 1x1 layer
 * with Ho, Wo >= 4 here (tile 8x8 when tile_h = 0), so all routes and
 * epilogues of a layer accumulate in the same order.  ksize: 1 or 3.
 * Tiles: 8x8, or 8x16 with stride 1 and ksize 3.  Other arguments as
 * cf_conv_mfma.  Replaces the same reference interfaces as cf_conv_mfma. */
int cf_conv_halo(const void* x, const void* w_packed, const float* alpha, const float* beta,
                 const float* v_in, float* v_out, float* out, void* out_nhwc, int64_t cp_out,
                 const float* identity, const void* identity_nhwc, int64_t cp_id,
                 int identity_mode, const int32_t* ag_mask, const int32_t* tile_order,
                 const unsigned long long* nnz, unsigned long long* nz_out,
                 const void* x_desc, const void* id_desc, void* out_desc, int bias_info,
                 const unsigned long long* id_nnz, int64_t numel, double sparse_threshold,
                 int64_t T,
                 int64_t B, int64_t Cp, int64_t Cout, int64_t Coutp, int64_t H, int64_t W, int64_t Ho, int64_t Wo,
                 int64_t ksize, int64_t stride, int64_t pad, int64_t tile_h, int64_t tile_w,
                 int64_t group_size, int epilogue, double tau, double v_th, double v_reset,
                 int hard_reset, int decay_input, void* stream);

/* A ResNet block's stride-2 3x3 conv1 (conv a, pad_a) and its stride-2 1x1
 * downsample (conv b, pad_b) of the same fp16 NHWC input x in one launch:
 * the workgroups of conv a's tiles, then conv b's, each computing exactly
 * what its own cf_conv_halo launch computes (same results, bit for bit),
 * reading x through the L2 once.  Both with the lean LIF epilogue: fp16
 * NHWC outputs out_a / out_b only (Cout a multiple of 32, no fp32 output,
 * no identity), v_in / v_out as cf_conv_mfma, their own count blocks nz_a /
 * nz_b, output descriptors desc_a / desc_b and bias knowledge
 * bias_info_a / bias_info_b (as out_desc / bias_info of cf_conv_mfma); the
 * input's count block nnz and descriptor x_desc (both nullable) route both
 * (StaticZero on a zero count or an all-zero copy); one set of LIF
 * parameters for both.  w/alpha/beta from
 * cf_pack_conv_weights.  Replaces the two launches of
 * catfuse/patterns.py:672-737 (SEWBasicBlock: conv1-bn1-sn1 and
 * downsample-downsample_sn of the same input). */
int cf_conv_halo_pair(const void* x, const unsigned long long* nnz, const void* x_desc,
                      int64_t numel, int64_t T, int64_t B, int64_t Cp, int64_t H, int64_t W,
                      int64_t Ho, int64_t Wo,
                      const void* w_a, const float* alpha_a, const float* beta_a,
                      const float* v_in_a, float* v_out_a, void* out_a, int64_t cp_out_a,
                      unsigned long long* nz_a, void* desc_a, int bias_info_a, int64_t Cout_a,
                      int64_t Coutp_a, int64_t pad_a,
                      const void* w_b, const float* alpha_b, const float* beta_b,
                      const float* v_in_b, float* v_out_b, void* out_b, int64_t cp_out_b,
                      unsigned long long* nz_b, void* desc_b, int bias_info_b, int64_t Cout_b,
                      int64_t Coutp_b, int64_t pad_b,
                      double tau, double v_th, double v_reset, int hard_reset, int decay_input,
                      void* stream);

/* cf_conv_mfma's and cf_conv_halo_pair's arguments as one block each, in
 * the order of their parameters, every field 8 bytes (the int parameters
 * as int64_t): the same launches for a caller whose per-call conversion of
 * 48 separate arguments costs more than the launch itself (a Python ctypes
 * binding re-filling a few fields of a block it keeps per layer).  No
 * counterpart in the reference (its Triton launches take Python arguments).
 * cf_conv_args_sizes writes sizeof of both blocks (sizes[0], sizes[1]) for
 * a binding to check its mirror of the layout. */
typedef struct CfConvMfmaArgs {
  const void* x;
  const void* w_packed;
  const float* alpha;
  const float* beta;
  const float* v_in;
  float* v_out;
  float* out;
  void* out_nhwc;
  int64_t cp_out;
  const float* identity;
  const void* identity_nhwc;
  int64_t cp_id;
  int64_t identity_mode;
  const int32_t* ag_mask;
  const int32_t* tile_order;
  const unsigned long long* nnz;
  unsigned long long* nz_out;
  const void* x_desc;
  const void* id_desc;
  void* out_desc;
  int64_t bias_info;
  const unsigned long long* id_nnz;
  int64_t numel;
  double sparse_threshold;
  int64_t T;
  int64_t B;
  int64_t Cp;
  int64_t Cout;
  int64_t Coutp;
  int64_t H;
  int64_t W;
  int64_t Ho;
  int64_t Wo;
  int64_t KH;
  int64_t KW;
  int64_t stride;
  int64_t pad;
  int64_t x_img_tstride;
  int64_t tile_h;
  int64_t tile_w;
  int64_t group_size;
  int64_t epilogue;
  double tau;
  double v_th;
  double v_reset;
  int64_t hard_reset;
  int64_t decay_input;
  void* stream;
} CfConvMfmaArgs;

typedef struct CfConvHaloPairArgs {
  const void* x;
  const unsigned long long* nnz;
  const void* x_desc;
  int64_t numel;
  int64_t T;
  int64_t B;
  int64_t Cp;
  int64_t H;
  int64_t W;
  int64_t Ho;
  int64_t Wo;
  const void* w_a;
  const float* alpha_a;
  const float* beta_a;
  const float* v_in_a;
  float* v_out_a;
  void* out_a;
  int64_t cp_out_a;
  unsigned long long* nz_a;
  void* desc_a;
  int64_t bias_info_a;
  int64_t Cout_a;
  int64_t Coutp_a;
  int64_t pad_a;
  const void* w_b;
  const float* alpha_b;
  const float* beta_b;
  const float* v_in_b;
  float* v_out_b;
  void* out_b;
  int64_t cp_out_b;
  unsigned long long* nz_b;
  void* desc_b;
  int64_t bias_info_b;
  int64_t Cout_b;
  int64_t Coutp_b;
  int64_t pad_b;
  double tau;
  double v_th;
  double v_reset;
  int64_t hard_reset;
  int64_t decay_input;
  void* stream;
} CfConvHaloPairArgs;

int cf_conv_mfma_args(const CfConvMfmaArgs* args);
int cf_conv_halo_pair_args(const CfConvHaloPairArgs* args);
int cf_conv_args_sizes(int64_t* sizes);

/* One-byte spike copies between fused layers.  The _u8 entry points take
 * and write NHWC copies of one byte per channel ([T*B][H][W][cp] uint8, the
 * same element layout as the fp16 copies, channels >= C zero): the spike
 * values the fused layers exchange (0/1, SEW sums, any integer 0..255) are
 * exact in a byte, and the byte copies halve the copies' HBM traffic.  The
 * conv entry points widen each staged byte to fp16 in LDS, so their K loop,
 * accumulation order and results are those of the fp16-copy entry points
 * bit for bit.  Replaces the fp32 -> uint8 spike exchange motivated by
 * tests/test_32_spike_uint8.py:16-104 (which casts fp32 spikes to uint8
 * between layers).
 *
 * cf_conv_halo_u8: cf_conv_halo with the lean LIF epilogue (no fp32 output,
 * identity only as a copy: identity_copy nullable, added to the spikes),
 * 8x8 tiles, Cout a multiple of 32, cp_out a multiple of 8, Cp of 32;
 * x / identity_copy / out_copy one byte per channel; other arguments as
 * cf_conv_halo.  cf_conv_halo_pair_u8: cf_conv_halo_pair on byte copies.
 * cf_conv_stem_lif_maxpool_u8: the stem writing its pooled output as a byte
 * copy (out_copy).  cf_nhwc_to_nchw_u8 / cf_global_avgpool_nhwc_u8: as the
 * fp16 forms, reading a byte copy.  cf_copy_u8_to_f16: a byte copy of n
 * elements (a multiple of 8) widened to an fp16 copy, for readers that take
 * fp16 copies only.  No other counterpart in the reference. */
int cf_conv_halo_u8(const void* x, const void* w_packed, const float* alpha, const float* beta,
                    const float* v_in, float* v_out, void* out_copy, int64_t cp_out,
                    const void* identity_copy, int64_t cp_id, const int32_t* ag_mask,
                    const int32_t* tile_order, const unsigned long long* nnz,
                    unsigned long long* nz_out, const void* x_desc, const void* id_desc,
                    void* out_desc, int bias_info, const unsigned long long* id_nnz,
                    int64_t numel, double sparse_threshold, int64_t T, int64_t B, int64_t Cp,
                    int64_t Cout, int64_t Coutp, int64_t H, int64_t W, int64_t Ho, int64_t Wo,
                    int64_t ksize, int64_t stride, int64_t pad, int64_t group_size, double tau,
                    double v_th, double v_reset, int hard_reset, int decay_input, void* stream);
int cf_conv_halo_pair_u8(const void* x, const unsigned long long* nnz, const void* x_desc,
                         int64_t numel, int64_t T, int64_t B, int64_t Cp, int64_t H, int64_t W,
                         int64_t Ho, int64_t Wo,
                         const void* w_a, const float* alpha_a, const float* beta_a,
                         const float* v_in_a, float* v_out_a, void* out_a, int64_t cp_out_a,
                         unsigned long long* nz_a, void* desc_a, int bias_info_a, int64_t Cout_a,
                         int64_t Coutp_a, int64_t pad_a,
                         const void* w_b, const float* alpha_b, const float* beta_b,
                         const float* v_in_b, float* v_out_b, void* out_b, int64_t cp_out_b,
                         unsigned long long* nz_b, void* desc_b, int bias_info_b, int64_t Cout_b,
                         int64_t Coutp_b, int64_t pad_b,
                         double tau, double v_th, double v_reset, int hard_reset,
                         int decay_input, void* stream);
int cf_conv_stem_lif_maxpool_u8(const float* x, const void* w_stem, const float* alpha,
                                const float* beta, const float* v_in, float* v_out, float* out,
                                void* out_copy, int64_t cp_out, uint32_t* status,
                                unsigned long long* nz_out, int64_t T, int64_t B, int64_t Cin,
                                int64_t Cout, int64_t Coutp, int64_t H, int64_t W, int64_t KH,
                                int64_t KW, int64_t stride, int64_t pad, int64_t pool_k,
                                int64_t pool_stride, int64_t pool_pad, double tau, double v_th,
                                double v_reset, int hard_reset, int decay_input, void* stream);
int cf_nhwc_to_nchw_u8(const void* xp, float* out, int64_t NB, int64_t C, int64_t H, int64_t W,
                       int64_t cp, void* stream);
int cf_global_avgpool_nhwc_u8(const void* xp, const void* desc, float* out, int64_t NB,
                              int64_t HW, int64_t C, int64_t cp, void* stream);
int cf_copy_u8_to_f16(const void* src, void* dst, int64_t n, void* stream);

/* A layer's response to its BN bias alone (the StaticZero drive z =
 * 0 * alpha + beta, alpha/beta from cf_pack_conv_weights, Cout entries;
 * pool = 1: the drive of cf_conv_mfma's pooled epilogue, the 2x2 average
 * (((z + z) + z) + z) * 0.25 of that z), from the initial state over T
 * steps, with the halo kernel's operations:
 * v_final [Cout] the final potential and fires [Cout] 1 where the channel
 * fires at some step.  Computed once per layer and T; the bias_info of
 * cf_conv_mfma states it.  No counterpart in the reference (its StaticZero
 * short-circuit, catfuse/implementations/base.py:250-308
 * static_zero_forward, broadcasts the bias and runs the LIF on every
 * call). */
int cf_bias_response(const float* alpha, const float* beta, int64_t Cout, int64_t T, int pool,
                     double tau, double v_th, double v_reset, int hard_reset, int decay_input,
                     float* v_final, uint32_t* fires, void* stream);

/* Fused Conv -> BN -> LIF / z in fp32 (VALU) for analog inputs
 * x [T*x_img_tstride + B][Cin][H][W]; x_img_tstride == 0 evaluates the
 * convolution once for a time-repeated (direct-encoded) input.  Replaces
 * catfuse/implementations/dense_keep.py:97-155 for the network stem. */
int cf_conv_direct(const float* x, const float* w, const float* alpha, const float* beta,
                   const float* v_in, float* v_out, float* out, void* out_nhwc, int64_t cp_out,
                   int64_t T, int64_t B,
                   int64_t Cin, int64_t Cout, int64_t H, int64_t W, int64_t Ho, int64_t Wo,
                   int64_t KH, int64_t KW, int64_t stride, int64_t pad, int64_t x_img_tstride,
                   int epilogue, double tau, double v_th, double v_reset, int hard_reset,
                   int decay_input, void* stream);

/* Conv(3 x 3, stride 1, Cin <= 4) -> BN -> LIF -> MaxPool2d(3, 2, 1) of an
 * analog input x [T*x_img_tstride + B][Cin][H][W] in one launch (fp32 VALU,
 * the same arithmetic as cf_conv_direct, so the pooled spikes equal
 * cf_conv_direct's followed by the pool bit for bit).  wt is the transposed
 * filter [Cin*9][Cout]; alpha/beta as cf_pack_conv_weights writes them.
 * Writes the pooled fp16 NHWC copy [T*B][Hp][Wp][cp_out] (channels
 * Cout .. cp_out-1 zero; cp_out a multiple of 8), the conv-resolution
 * membrane v_out [B][Cout][Ho][Wo] (nullable), and publishes the output's
 * count block nz_out (nullable; see the count-block convention above).
 * Replaces the first stage of the reference's spiking patch splitter,
 * models/spikformer_github.py:181-254 (proj_conv, proj_bn, proj_lif, maxpool),
 * which runs the conv, the LIF and the pool as separate passes. */
int cf_conv_direct_lif_maxpool(const float* x, const float* wt, const float* alpha,
                               const float* beta, const float* v_in, float* v_out,
                               void* out_nhwc, int64_t cp_out, unsigned long long* nz_out,
                               int64_t T, int64_t B, int64_t Cin, int64_t Cout, int64_t H,
                               int64_t W, int64_t pad, int64_t x_img_tstride, double tau,
                               double v_th, double v_reset, int hard_reset, int decay_input,
                               void* stream);

/* Conv(3 x 3, stride 1, Cin <= 4) -> BN -> AvgPool2d(2, 2) -> LIF of an
 * analog input x [T*x_img_tstride + B][Cin][H][W] in one launch (fp32 VALU,
 * the arithmetic of cf_conv_direct, then the pool sum
 * ((z00 + z01) + z10) + z11 times 0.25 and the LIF of cf_avgpool2x2_lif, so
 * the spikes equal cf_conv_direct (epilogue 1) followed by
 * cf_avgpool2x2_lif bit for bit; a stride-0 time axis evaluates the conv
 * once).  wt is the transposed filter [Cin*9][Cout]; alpha/beta as for
 * cf_conv_direct; Cout a multiple of 16.  Writes the pooled fp16 NHWC copy
 * [T*B][Hp][Wp][cp_out] (Hp = Ho / 2, Wp = Wo / 2; channels Cout ..
 * cp_out-1 zero; cp_out a multiple of 8) and the pooled membrane v_out
 * [B][Cout][Hp][Wp] (nullable; v_in likewise), and publishes the output's
 * count block nz_out (nullable).  Replaces the reference's F8
 * (catfuse/kernels/conv_pool_lif.py:94-178: the conv's z written to HBM, then
 * the pool and the LIF) for the first layer of a spiking VGG. */
int cf_conv_direct_avgpool_lif(const float* x, const float* wt, const float* alpha,
                               const float* beta, const float* v_in, float* v_out,
                               void* out_nhwc, int64_t cp_out, unsigned long long* nz_out,
                               int64_t T, int64_t B, int64_t Cin, int64_t Cout, int64_t H,
                               int64_t W, int64_t pad, int64_t x_img_tstride, double tau,
                               double v_th, double v_reset, int hard_reset, int decay_input,
                               void* stream);

/* Stem weight packing for cf_conv_stem_lif_maxpool: fp32 [Cout][Cin][KH][KW]
 * (Cin <= 4, KH <= 7, KW <= 8) -> fp16 hi/lo limbs [2][Coutp][KH][32] with
 * k = kw*4 + c, a per-channel power-of-two prescale, and the folded
 * epilogue alpha/beta [Coutp] (BN scale/shift, conv bias).  Replaces the
 * weight handling of catfuse/implementations/dense_keep.py:73-95 for the
 * stem. */
int cf_pack_stem_weights(const float* w, int64_t Cout, int64_t Cin, int64_t KH, int64_t KW,
                         int64_t Coutp, const float* bn_scale, const float* bn_shift,
                         const float* bias, void* w_stem, float* alpha, float* beta,
                         void* stream);

/* Fused stem Conv(stride 2 or 1) -> BN -> LIF -> MaxPool2d(3, 2, 1) on the
 * matrix cores for a direct-encoded image x [B][Cin][H][W] (the same frame at all T
 * <= 32 steps: the conv runs once, its z feeds every LIF step).  The image
 * is split into fp16 hi/lo limbs; products wh*xh + wl*xh + wh*xl accumulate
 * in fp32.  Outputs the pooled spikes out [T][B][Cout][Hp][Wp] and/or their
 * fp16 NHWC copy [T*B][Hp][Wp][cp_out]; v_in/v_out hold the
 * conv-resolution membrane channels-last, [B][Hc][Wc][Cout] (a conv output's
 * channels contiguous: 16-byte state accesses; torch's channels_last format
 * of a [B, Cout, Hc, Wc] tensor).  status |= 2 if |x| > 65504 or not finite.
 * nz_out (nullable): the pooled output's count block (see the count-block
 * convention above).  Replaces catfuse/implementations/dense_keep.py:97-155
 * (conv1/bn1/sn1 via catfuse/patterns.py:237-387) plus the unfused
 * SpikingJelly MaxPool2d that follows it in the ResNet stem (stride 2), and
 * the first stage of the Spikformer patch splitter,
 * models/spikformer_github.py:181-254 (stride 1). */
int cf_conv_stem_lif_maxpool(const float* x, const void* w_stem, const float* alpha,
                             const float* beta, const float* v_in, float* v_out, float* out,
                             void* out_nhwc, int64_t cp_out, uint32_t* status,
                             unsigned long long* nz_out, int64_t T,
                             int64_t B, int64_t Cin, int64_t Cout, int64_t Coutp, int64_t H,
                             int64_t W, int64_t KH, int64_t KW, int64_t stride, int64_t pad,
                             int64_t pool_k, int64_t pool_stride, int64_t pool_pad, double tau,
                             double v_th, double v_reset, int hard_reset, int decay_input,
                             void* stream);

/* Fused grouped Conv -> BN -> LIF (groups > 1; depthwise when groups == Cin)
 * over T steps, one streaming launch (a grouped conv is HBM-bound).  Input:
 * exactly one of x, fp16 NHWC [T*B][H][W][Cp] (channels >= Cin zero; Cp a
 * multiple of 8), or x32, fp32 NCHW [T*x_img_tstride + B][Cin][H][W]
 * (x_img_tstride 0: the same image at every step).  w fp32
 * [Cout][Cin/groups][ksize][ksize]; alpha/beta [Cout] as cf_pack_conv_weights
 * writes them with w_packed NULL; v_in/v_out channels-last [B][Ho][Wo][Cout]
 * (nullable); out_nhwc fp16 [T*B][Ho][Wo][cp_out] (channels >= Cout zero);
 * nnz (nullable): the input's count block, zero -> StaticZero (no input
 * reads); nz_out (nullable): the output's count block.  Each output sums
 * its group's products in fp32 in the order kh, kw, input channel.
 * Replaces catfuse/sparseflow/sparse_grouped_conv2d_kernel.py:93-364
 * (sparse_grouped_conv2d_forward: groups as independent sparse conv
 * sub-problems), with BN and the LIF of the layer fused. */
int cf_conv_grouped_lif(const void* x, const float* x32, int64_t x_img_tstride, const float* w,
                        const float* alpha, const float* beta, const float* v_in, float* v_out,
                        void* out_nhwc, int64_t cp_out, const unsigned long long* nnz,
                        unsigned long long* nz_out, int64_t T, int64_t B, int64_t Cin, int64_t Cp,
                        int64_t Cout, int64_t groups, int64_t H, int64_t W, int64_t Ho,
                        int64_t Wo, int64_t ksize, int64_t stride, int64_t pad, double tau,
                        double v_th, double v_reset, int hard_reset, int decay_input,
                        void* stream);

/* Library error code returned beside the hipError_t values: the input of
 * cf_conv_sparse_noalloc needs more workspace than its static array holds. */
#define CF_ERROR_NOALLOC_LIMIT 7001

/* Workspace of cf_conv_sparse_noalloc, a static device array of
 * CF_NOALLOC_SCRATCH_BYTES (about 9.5 MiB) on every GPU the library runs on:
 * the input's count block, activity bits for up to CF_NOALLOC_MAX_PIXELS
 * input pixels (T*B*H*W), tile masks for up to CF_NOALLOC_MAX_TILES
 * prescan tiles (T*B*ceil(Ho/tile_h)*ceil(Wo/tile_w)) and their compacted
 * order. */
#define CF_NOALLOC_MAX_PIXELS (1 << 21)
#define CF_NOALLOC_MAX_TILES (1 << 17)
#define CF_NOALLOC_SCRATCH_BYTES (4096 + 4 * CF_NOALLOC_MAX_PIXELS + 12 * CF_NOALLOC_MAX_TILES + 256)

/* The SparseFlow-routed fused Conv -> BN -> LIF of cf_conv_mfma on an fp16
 * NHWC input (x [T*B][H][W][Cp], channels >= Cin zero, e.g. a fused conv's
 * output copy), with the routing workspace in the library instead of the
 * caller's memory: no allocation at all.  No counterpart in the reference;
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  It runs
 * cf_scan_nhwc (activity bits + nonzero count of x), cf_prescan_tiles (tile
 * masks, tile_h x tile_w output tiles, group_size-channel groups),
 * cf_compact_tiles and cf_conv_mfma routed on them (StaticZero / SparseFlow above
 * sparse_threshold / dense), with their workspace in a static device array
 * (CF_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends); results
 * are those of the same calls with caller buffers, bit for bit.
 * Square kernels (ksize x ksize); other arguments as cf_conv_mfma.  Returns
 * CF_ERROR_NOALLOC_LIMIT, launching nothing, when T*B*H*W >
 * CF_NOALLOC_MAX_PIXELS or the tile count > CF_NOALLOC_MAX_TILES.  Every
 * call on one GPU uses that GPU's array: calls that overlap on one GPU (on
 * streams not ordered against each other) race. */
int cf_conv_sparse_noalloc(const void* x, int64_t Cin, const void* w_packed, const float* alpha,
                           const float* beta, const float* v_in, float* v_out, float* out,
                           void* out_nhwc, int64_t cp_out, const float* identity,
                           const void* identity_nhwc, int64_t cp_id, int identity_mode,
                           unsigned long long* nz_out, double sparse_threshold, int64_t T,
                           int64_t B, int64_t Cp, int64_t Cout, int64_t Coutp, int64_t H,
                           int64_t W, int64_t Ho, int64_t Wo, int64_t ksize, int64_t stride,
                           int64_t pad, int64_t tile_h, int64_t tile_w, int64_t group_size,
                           int epilogue, double tau, double v_th, double v_reset, int hard_reset,
                           int decay_input, void* stream);

/* Diagnostic: one wave computes D(32x32 fp32) = A(32x16 fp16) * B(16x32
 * fp16) through the matrix-core lane mapping cf_conv_mfma relies on.
 * No reference counterpart (layout self-test). */
int cf_probe_mfma_layout(const void* A, const void* B, float* D, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CATFUSE_AMD_H */
