// gemm_kernels.hpp -- host launchers of the GEMM kernels (internal).
#pragma once
#include <hip/hip_runtime.h>

#include "gemm_common.hpp"

namespace lava {

// Any layout, any shape; C row-major with ldc.  OutT / EPI: the output type and the
// fused epilogue (see Epilogue); <T, acc type, false> is the plain GEMM.
template <typename T, typename OutT, bool EPI>
int launch_gemm_staged(const T* A, const T* B, OutT* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                       int64_t ldc, bool arow, bool brow, hipStream_t s, const Epilogue& epi);

// Products the 256 x 256 tile kernel would run on few CUs or on mostly empty tiles, on 64 x 64
// tiles (16 times the workgroups): at most SMALL_GEMM_MAX_TILES 256 x 256 tiles, and any product
// where the small kernel's estimated rate is the higher (small_gemm_preferred).
// small_gemm_fits() says whether the layout fits the kernel's 16-byte chunks (C row-major;
// arow / brow: A / B row-major).
constexpr int64_t SMALL_GEMM_MAX_TILES = 16;
template <typename T>
bool small_gemm_preferred(int64_t M, int64_t N, int64_t K);
template <typename T>
bool small_gemm_fits(const void* A, const void* B, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, bool arow,
                     bool brow);
template <typename T, typename OutT, bool EPI>
int launch_gemm_small(const T* A, const T* B, OutT* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                      int64_t ldc, bool arow, bool brow, hipStream_t s, const Epilogue& epi);

// Split K for the small kernel's plain products (no epilogue): a product of at most 256 64 x 64
// tiles and at least 8 K chunks of 512 bytes (16 above 128 tiles) runs in `splits` K ranges of kspan elements (each
// >= 2 chunks, splits x tiles <= 512, splits <= SMALL_GEMM_MAX_SPLITS) whose partial products go
// to the stream's workspace and are summed in split order into C by a second kernel.
constexpr int64_t SMALL_GEMM_MAX_SPLITS = 16;
struct SmallSplit {
    int splits = 1;
    int64_t kspan = 0;
};
template <typename T>
SmallSplit small_gemm_splits(int64_t M, int64_t N, int64_t K);
// Workspace bytes of a split plan: the W8A16 counter region, then one M x N partial per split.
template <typename T>
size_t small_splitk_bytes(int64_t M, int64_t N, const SmallSplit& sp);
// U8: int8 storage read as unsigned bytes (uint32 results in the int32 words).
template <typename T, bool U8 = false>
int launch_gemm_small_splitk(const T* A, const T* B, typename Mfma16<T>::acc_elem* C, int64_t M, int64_t N, int64_t K,
                             int64_t lda, int64_t ldb, int64_t ldc, bool arow, bool brow, void* stream,
                             const SmallSplit& sp);
// Unsigned bytes on the small kernel, unsplit (flipped bytes, signed MFMAs, row / column sums).
int launch_gemm_small_u8(const int8_t* A, const int8_t* B, int32_t* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                         int64_t ldb, int64_t ldc, bool arow, bool brow, hipStream_t s);

// The 16x16x16 vocabulary-tile GEMM (fp16 -> fp32); M, N, K multiples of 16.
int launch_coopmat_tiles(const f16* A, const f16* B, float* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                         int64_t ldb, int64_t ldc, uint32_t layout, hipStream_t s);

// The fast path, C row-major: A and B each K-contiguous (A row-major, B column-major)
// or, for 16-bit types, M/N-contiguous (A column-major, B row-major).
// tn_gemm_eligible() says whether it applies: TN_FULL for whole 256 x 256 tiles and
// 64-element K steps, TN_RAGGED for other extents (a K-contiguous operand needs K a
// multiple of 16 bytes, an M/N-contiguous one M or N a multiple of 8).
enum TnFit : int { TN_NO = 0, TN_FULL = 1, TN_RAGGED = 2 };
template <typename T>
int tn_gemm_eligible(const void* A, const void* B, const void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                     int64_t ldb, int64_t ldc, size_t c_elem, bool ak, bool bk);
template <typename T, typename OutT, bool EPI>
int launch_gemm_tn(const T* A, const T* B, OutT* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                   int64_t ldc, hipStream_t s, const Epilogue& epi, bool ragged, bool ak, bool bk);
// Unsigned bytes x unsigned bytes -> uint32 (wrapped) on the tile kernel: signed MFMAs on the
// bytes flipped by 128, corrected by the row and column sums (gemm_tn_kernel.hpp).
int launch_gemm_tn_u8(const int8_t* A, const int8_t* B, int32_t* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                      int64_t ldb, int64_t ldc, hipStream_t s, bool ragged, bool ak, bool bk);
// The mid-size kernel (gemm_mid_kernel.hpp): 128 x 128 tiles, two workgroups per CU; f16 / bf16 /
// int8, each operand K- or M/N-contiguous (ak: A row-major, bk: B column-major); fp32 / int32 output,
// or (EPI, f16 / bf16) the fused epilogue into OutT, or (U8) unsigned bytes into uint32 words.  mid_gemm_eligible() gives TN_FULL (whole
// tiles and 128-byte K steps, C rows of 4 c_elem-byte elements aligned), TN_RAGGED (any extents: K
// a multiple of the 16-byte chunk for a K-contiguous operand, M or N of it for an M/N-contiguous one)
// or TN_NO.
template <typename T>
int mid_gemm_eligible(const void* A, const void* B, const void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                      int64_t ldb, int64_t ldc, size_t c_elem, bool ak, bool bk);
template <typename T, typename OutT, bool EPI, bool U8 = false>
int launch_gemm_mid(const T* A, const T* B, OutT* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                    int64_t ldc, hipStream_t s, const Epilogue& epi, bool ragged, bool ak, bool bk);
// Whether an M x N product takes the mid-size kernel when it fits (the measured choice against the
// tile and small-product kernels).
bool mid_gemm_preferred(int64_t M, int64_t N);
// Any shape and layout: one thread per element of C, bytes widened and summed in uint32.
int launch_gemm_u8_generic(const uint8_t* A, const uint8_t* B, uint32_t* C, int64_t M, int64_t N, int64_t K,
                           int64_t lda, int64_t ldb, int64_t ldc, uint32_t layout, hipStream_t s);

}  // namespace lava
