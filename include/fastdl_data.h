/*
 * fastdl_data.h -- C-ABI of the MI355X (gfx950) input side of the MLP path:
 * IDX (MNIST) bytes resident in HBM, turned into the fp32 batch and int64
 * labels that fdl_mlp2_train_step consumes.
 *
 * Conventions as in fastdl_gemm.h: plain C, device pointers on the calling
 * thread's current HIP device, `stream` is a hipStream_t passed as void*
 * (NULL = null stream), no allocation, asynchronous, negative fdl_status
 * codes on failure with fdl_last_error() holding the message.
 */
#ifndef FASTDL_DATA_H
#define FASTDL_DATA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Gather `batch` rows of a row-major byte matrix (images: count rows of
 * row_bytes pixels each) into fp32, and their labels into int64:
 *
 *   r = index ? index[b] : b                      for b in [0, batch)
 *   x[b * row_bytes + j] = (float)images[r * row_bytes + j] / divisor
 *   y[b] = (int64_t)(int8_t)labels[r]
 *
 * Replaces the pixel and label conversion of the legacy MNIST loader
 * (legacy/src/data/DataLoader.cpp:61-68 divides each pixel by 255.0f;
 * :87-90 reads each label through a plain `char`, which is signed on the
 * x86-64 hosts the reference builds on, hence the int8 sign extension).
 * The division is IEEE round-to-nearest, so with divisor = 255 the bits equal
 * the reference's host conversion.  index == NULL gathers rows 0..batch-1,
 * which converts the whole set in one launch (the reference's
 * getImagesMatrix).  index is a device array of batch int64 row numbers; an
 * entry outside [0, count) yields a row of zeros and label -1 (a label that
 * fdl_softmax_xent and fdl_mlp2_train_step leave out of the loss), so a bad
 * index never reads outside the inputs.
 *
 * x may be NULL (labels only) when y is not, and y may be NULL (pixels only);
 * images and labels may be NULL when count == 0 (every row is then out of
 * range) or when x, respectively y, is NULL.  Without an index, batch must
 * not exceed count.  batch == 0 is a no-op.  divisor must be finite and
 * non-zero.
 */
int fdl_idx_gather(const uint8_t* images, const uint8_t* labels, int64_t count,
                   int64_t row_bytes, const int64_t* index, int64_t batch,
                   float divisor, float* x, int64_t* y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FASTDL_DATA_H */
