/*
 * oracle.h - ORACLE (test infrastructure only): CPU restatement of the
 * reference's conv / GEMM path and a CPU runner for ENNF models. Used by the
 * tests as the parity reference and by bench.py as the timed CPU baseline;
 * never linked into the product library.
 */
#ifndef SPINN_ORACLE_H
#define SPINN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

typedef struct {
    int n, c, h, w, oc, oh, ow, kh, kw, sh, sw, ph, pw, group, act;
} OracleConv;

void oracle_set_as_shipped(int on);
float *oracle_pack_a(int M, int K, const float *A, int lda);
void oracle_sgemm_packed(int M, int N, int K, const float *pa, const float *B, int ldb, float *C, int ldc);
void oracle_sgemm(int M, int N, int K, float alpha, const float *A, int lda, const float *B, int ldb, float beta,
                  float *C, int ldc);
int oracle_conv2d(const OracleConv *p, const float *X, const float *W, const float *bias, const float *R, float *Y);
int oracle_conv2d_f64(const OracleConv *p, const float *X, const float *W, const float *bias, const float *R,
                      double *Y);
int oracle_winograd(const OracleConv *p, const float *X, const float *W, const float *bias, const float *R, float *Y);
int oracle_gemm(int M, int N, int K, int transA, int transB, float alpha, float beta, const float *A, const float *B,
                const float *C, int c_elems, float *Y);
int oracle_gemm_f64(int M, int N, int K, int transA, int transB, double alpha, double beta, const float *A,
                    const float *B, const float *C, int c_elems, double *Y);
int oracle_matmul(int batch, int M, int N, int K, const float *A, const float *B, float *Y);
void oracle_maxpool(int N, int C, int H, int W, int OH, int OW, int KH, int KW, int SH, int SW, int PH, int PW,
                    const float *X, float *Y);
void oracle_reduce_mean(long outer, long dim, long inner, const float *X, float *Y);
void oracle_binary(int op, const float *a, uint32_t na, const float *b, uint32_t nb, float *y, uint32_t n);
void oracle_unary(int op, const float *x, float *y, long n);
void oracle_batchnorm(long N, long C, long spatial, const float *X, const float *scale, const float *bias,
                      const float *mean, const float *var, float eps, float *Y);
void oracle_softmax(long outer, long dim, long inner, const float *X, float *Y);
void oracle_concat(int n_in, const float *const *xs, const long *sizes, long outer, long inner, float *Y);
void oracle_split(int n_out, float *const *ys, const long *sizes, long outer, long inner, const float *X);
void oracle_transpose(int ndim, const long *dims, const int *perm, const float *X, float *Y);
void oracle_resize_nearest(long planes, int H, int W, int OH, int OW, const float *X, float *Y);
void oracle_reduce_max(uint32_t out_n, uint32_t block, const float *X, float *Y);
int oracle_topk(long rows, long n, long k, const float *X, float *vals, int64_t *idx);
void oracle_gather_elements(int ndim, const uint32_t *in_dims, const uint32_t *out_dims, int axis,
                            const float *data, const void *indices, int index_dtype, float *Y, uint32_t n);
void oracle_tile(int ndim, const uint32_t *in_dims, const uint32_t *out_dims, int elem_size, const void *X,
                 void *Y);
int oracle_cast(int src, int dst, uint32_t n, const void *X, void *Y);
int oracle_binary_typed(int op, int dtype, const void *a, uint32_t na, const void *b, uint32_t nb, void *y,
                        uint32_t n);
int oracle_num_threads(void);
void oracle_set_num_threads(int n);

/* CPU model runner over an ENNF file (oracle/cpu_runtime.c). */
typedef struct OracleModel OracleModel;
OracleModel *oracle_model_load(const char *path);
int oracle_model_run(OracleModel *m, const float *input, float *output);
int oracle_model_num_nodes(const OracleModel *m);
/* Copy tensor `id` of the last run (activation or weight) into `dst`; returns bytes copied or -1. */
long oracle_model_tensor(const OracleModel *m, int id, void *dst, size_t bytes);
/* Use the Winograd restatement for eligible 3x3 stride-1 convolutions (0 = im2col path). */
void oracle_model_set_winograd(OracleModel *m, int on);
void oracle_model_free(OracleModel *m);

#endif
