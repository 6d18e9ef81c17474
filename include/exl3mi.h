/* exl3mi: EXL3 trellis-quantized linear and grouped-MoE kernels for AMD Instinct MI355X (gfx950).
 *
 * Plain C ABI: device pointers, sizes, a hipStream_t passed as void*. Every entry point is asynchronous on `stream`
 * (NULL = the default stream), never synchronises the host, and returns an exl3_status. The caller owns every input
 * and output buffer; outputs are written in place. Library-owned scratch is cached per device (grown on demand; see
 * exl3_reserve_workspace). Calls on one device must be ordered on one stream.
 *
 * Data formats (identical to exllamav3 / the reference, ext-op-inventory.md:698-777):
 *   trellis  int16 [k/16][n/16][16*K], K = bits per weight (1..8), one 16x16 tile = 8*K little-endian uint32 words
 *   suh      fp16 [k], svh fp16 [n] (sign flips with the channel scales folded in)
 *   W = diag(suh) Hblk W_hat Hblk diag(svh), Hblk = blockdiag(H128 / sqrt(128)); y = x @ W
 * Codebook: only cb = 2 (mul1, the codebook every checkpoint of the reference uses) is implemented.
 */
#ifndef EXL3MI_H
#define EXL3MI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EXL3_ABI_VERSION 1

enum exl3_status {
    EXL3_OK = 0,
    EXL3_ERR_INVALID = 1,     /* bad shape, dtype, alignment or pointer: the reference's TORCH_CHECK -> RuntimeError */
    EXL3_ERR_UNSUPPORTED = 2, /* K / codebook / mode not implemented: NotImplementedError */
    EXL3_ERR_HIP = 3          /* HIP runtime error */
};

enum exl3_dtype { EXL3_F16 = 0, EXL3_F32 = 1 };
enum exl3_act { EXL3_ACT_SILU = 0, EXL3_ACT_GELU_TANH = 1 };

/* Message for the last non-zero status returned on the calling thread. */
const char* exl3_last_error(void);
int exl3_abi_version(void);

/* Pre-size this device's workspace (bytes of scratch, number of arrival counters) so later calls do not allocate,
 * e.g. before HIP graph capture. No reference counterpart (the reference grows its scratch inside the op). */
int exl3_reserve_workspace(int64_t bytes, int64_t ncounters);

/* Decoded Hadamard-domain weight slice: out[r, c] = W_hat[r, n_offset + c] (fp16 bits, row stride out_ld elements),
 * no sign vectors applied. Bit-exact with the reference decode.
 * Replaces: exllamav3 ext reconstruct / reconstruct_slice (ext-op-inventory.md:597-612) and
 *           exl3xpu_C::exl3_reconstruct (glm/xpu/csrc/exl3_ops.sycl:539-555, bound at :791-799).
 * k % 16 == 0, n_total % 16 == 0, n_offset and n_slice multiples of 128, n_offset + n_slice <= n_total. */
int exl3_reconstruct(const int16_t* trellis, int64_t k, int64_t n_total, int K, int cb, int64_t n_offset,
                     int64_t n_slice, uint16_t* out, int64_t out_ld, void* stream);

/* Blockwise 128-point Hadamard: out[r, blk] = (H128 @ (in[r, blk] (* pre))) * scale / sqrt(128) (* post).
 * in/out [rows, cols] with row strides in_ld/out_ld, both of `dtype`; cols % 128 == 0; in-place allowed.
 * pre/post fp16 [cols] or NULL; if both are given only pre is applied. fp16 path rounds x*pre, the scaled sum and
 * the *post product to fp16; the fp32 path does not round.
 * Replaces: exllamav3 ext had_r_128 (ext-op-inventory.md:576-595; glm/xpu/glm_xpu/ops.py:130-142). */
int exl3_had_r_128(const void* in, int64_t in_ld, void* out, int64_t out_ld, int64_t rows, int64_t cols, int dtype,
                   const uint16_t* pre, const uint16_t* post, float scale, void* stream);

/* EXL3 linear: C[m, n] = Hn( Hk(A * suh) @ W_hat ) * svh for A fp16 [m, k] (row stride a_ld), C fp16 or fp32
 * [m, n] (row stride c_ld). A_had (fp16 scratch, >= m*k elements) is accepted for signature compatibility and not
 * used: the input transform is fused. cb must be 2 (mul1).
 * Replaces: exllamav3 ext exl3_gemm(A, B, C, suh, A_had, svh, force_shape_idx, mcg, mul1, force_num_sms)
 *           (ext-op-inventory.md:498-557) and exl3xpu_C::exl3_gemm_small / linear (glm/xpu/csrc/exl3_ops.sycl:258-321,
 *           643-757). */
int exl3_gemm(const uint16_t* A, int64_t a_ld, int64_t m, int64_t k, const int16_t* B, int64_t n, int K, void* C,
              int64_t c_ld, int c_dtype, const uint16_t* suh, uint16_t* A_had, const uint16_t* svh, int cb,
              void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EXL3MI_H */
