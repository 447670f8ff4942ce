/*
 * xgboost_c_api.h -- the drop-in boundary of the HIP hist engine.
 *
 * These are the XGBoost C API entry points that the Python package
 * (`import xgboost as xgb`) binds over ctypes for DMatrix/QuantileDMatrix,
 * train, Booster and the sklearn estimators with tree_method='hist'.  Each
 * declaration keeps the upstream signature and names the reference
 * implementation it replaces (src/c_api.cpp of tabulai/xgboost-metal; upstream
 * declarations in include/xgboost/c_api.h).
 *
 * Conventions (src/c_api.cpp:17-40): every function returns 0 on success and
 * -1 on failure, with the message in XGBGetLastError(); handles are opaque
 * pointers owned by the caller and released with XG*Free; strings and arrays
 * returned through out-pointers stay valid until the next call on the same
 * thread; booster calls are serialised per booster.
 */
#ifndef XGBOOST_HIP_C_API_H
#define XGBOOST_HIP_C_API_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
#define XGB_EXTERN_C extern "C"
#else
#define XGB_EXTERN_C
#endif
#define XGB_DLL XGB_EXTERN_C __attribute__((visibility("default")))

typedef uint64_t bst_ulong;
typedef void* DMatrixHandle;
typedef void* BoosterHandle;
typedef void* DataIterHandle;
typedef void* TrackerHandle;
typedef void* CategoriesHandle;
/* Data iterator callbacks (upstream include/xgboost/c_api.h): reset rewinds
 * the iterator; next sets the next batch on the proxy DMatrix and returns 1,
 * or returns 0 at the end. */
typedef void DataIterResetCallback(DataIterHandle handle);
typedef int XGDMatrixCallbackNext(DataIterHandle iter);

/* --- library ------------------------------------------------------------ */
XGB_DLL const char* XGBGetLastError(void);                       /* c_api.cpp:176 */
XGB_DLL void XGBoostVersion(int* major, int* minor, int* patch);  /* c_api.cpp:175 */
XGB_DLL int XGBuildInfo(char const** out);                        /* c_api.cpp:169-177 */
XGB_DLL int XGBRegisterLogCallback(void (*callback)(const char*)); /* c_api.cpp:169-177 */
XGB_DLL int XGBSetGlobalConfig(char const* config);               /* c_api.cpp:179-189 */
XGB_DLL int XGBGetGlobalConfig(char const** out_config);          /* c_api.cpp:179-189 */

/* --- DMatrix ------------------------------------------------------------ */
XGB_DLL int XGDMatrixCreateFromDense(char const* data, char const* config, DMatrixHandle* out); /* c_api.cpp:192-194 */
XGB_DLL int XGDMatrixCreateFromMat(const float* data, bst_ulong nrow, bst_ulong ncol, float missing,
                                   DMatrixHandle* out);                                          /* c_api.cpp:192 */
XGB_DLL int XGDMatrixCreateFromCSR(char const* indptr, char const* indices, char const* data, bst_ulong ncol,
                                   char const* config, DMatrixHandle* out);                      /* c_api.cpp:198 */
XGB_DLL int XGDMatrixFree(DMatrixHandle handle);                                                 /* c_api.cpp:213 */
XGB_DLL int XGDMatrixSetInfoFromInterface(DMatrixHandle handle, char const* field, char const* data); /* c_api.cpp:242 */
XGB_DLL int XGDMatrixSetFloatInfo(DMatrixHandle handle, const char* field, const float* array, bst_ulong len);
XGB_DLL int XGDMatrixGetFloatInfo(const DMatrixHandle handle, const char* field, bst_ulong* out_len,
                                  const float** out_dptr);
XGB_DLL int XGDMatrixSetStrFeatureInfo(DMatrixHandle handle, const char* field, const char** features,
                                       const bst_ulong size);
XGB_DLL int XGDMatrixGetStrFeatureInfo(DMatrixHandle handle, const char* field, bst_ulong* size,
                                       const char*** out_features);
XGB_DLL int XGDMatrixNumRow(DMatrixHandle handle, bst_ulong* out);                                /* c_api.cpp:274 */
XGB_DLL int XGDMatrixNumCol(DMatrixHandle handle, bst_ulong* out);                                /* c_api.cpp:275 */
XGB_DLL int XGDMatrixNumNonMissing(DMatrixHandle handle, bst_ulong* out);
/* Other host layouts, converted on ingest: CSC and COO to CSR (c_api.cpp:201-206),
 * columnar (a JSON list of per-column array interfaces) to dense (:195). */
XGB_DLL int XGDMatrixCreateFromCSC(char const* indptr, char const* indices, char const* data, bst_ulong nrow,
                                   char const* config, DMatrixHandle* out);
XGB_DLL int XGDMatrixCreateFromCOO(char const* row_idx, char const* col_idx, char const* data, bst_ulong nrow,
                                   bst_ulong ncol, char const* config, DMatrixHandle* out);
XGB_DLL int XGDMatrixCreateFromColumnar(char const* data, char const* config, DMatrixHandle* out);
/* Iterator ingestion (c_api.cpp:214-239): the proxy holds one batch at a time;
 * the batches are appended in order.  The QuantileDMatrix variant takes its
 * cuts from `ref` (a DMatrix handle) when given, else sketches its own with
 * config's max_bin. */
XGB_DLL int XGProxyDMatrixCreate(DMatrixHandle* out);
XGB_DLL int XGProxyDMatrixSetDataDense(DMatrixHandle handle, char const* data);
XGB_DLL int XGProxyDMatrixSetDataColumnar(DMatrixHandle handle, char const* data);
XGB_DLL int XGProxyDMatrixSetDataCSR(DMatrixHandle handle, char const* indptr, char const* indices, char const* data,
                                     bst_ulong ncol);
XGB_DLL int XGDMatrixCreateFromCallback(DataIterHandle iter, DMatrixHandle proxy, DataIterResetCallback* reset,
                                        XGDMatrixCallbackNext* next, char const* config, DMatrixHandle* out);
XGB_DLL int XGQuantileDMatrixCreateFromCallback(DataIterHandle iter, DMatrixHandle proxy, DataIterHandle ref,
                                                DataIterResetCallback* reset, XGDMatrixCallbackNext* next,
                                                char const* config, DMatrixHandle* out);
/* Rows idxset[0..len) of a matrix with their meta info (c_api.cpp:294-297). */
XGB_DLL int XGDMatrixSliceDMatrixEx(DMatrixHandle handle, int const* idxset, bst_ulong len, DMatrixHandle* out,
                                    int allow_groups);
XGB_DLL int XGDMatrixSliceDMatrix(DMatrixHandle handle, int const* idxset, bst_ulong len, DMatrixHandle* out);
/* The non-missing values as CSR into caller buffers sized by num_row + 1 and
 * XGDMatrixNumNonMissing (c_api.cpp:313). */
XGB_DLL int XGDMatrixGetDataAsCSR(DMatrixHandle handle, char const* config, bst_ulong* out_indptr,
                                  unsigned* out_indices, float* out_data);
/* label / weight / base_margin as an array-interface JSON string (c_api.cpp:255). */
XGB_DLL int XGDMatrixGetInfoRef(DMatrixHandle handle, char const* field, char const** out);
XGB_DLL int XGDMatrixWasZeroCopied(DMatrixHandle handle, int* out);  /* always 0: input is copied */
/* Cut points as two array-interface JSON strings (c_api.cpp:358). */
XGB_DLL int XGDMatrixGetQuantileCut(DMatrixHandle const handle, char const* config, char const** out_indptr,
                                    char const** out_data);

/* --- Booster ------------------------------------------------------------ */
XGB_DLL int XGBoosterCreate(const DMatrixHandle dmats[], bst_ulong len, BoosterHandle* out);     /* c_api.cpp:442-452 */
XGB_DLL int XGBoosterFree(BoosterHandle handle);
XGB_DLL int XGBoosterReset(BoosterHandle handle);                                                /* c_api.cpp:454-463 */
XGB_DLL int XGBoosterSetParam(BoosterHandle handle, const char* name, const char* value);         /* c_api.cpp:464 */
XGB_DLL int XGBoosterSetParams(BoosterHandle handle, char const* config);                        /* c_api.cpp:465-483 */
XGB_DLL int XGBoosterUpdateOneIter(BoosterHandle handle, int iter, DMatrixHandle dtrain);        /* c_api.cpp:484 */
XGB_DLL int XGBoosterBoostOneIter(BoosterHandle handle, DMatrixHandle dtrain, float* grad, float* hess,
                                  bst_ulong len);
XGB_DLL int XGBoosterTrainOneIter(BoosterHandle handle, DMatrixHandle dtrain, int iter, char const* grad,
                                  char const* hess);
XGB_DLL int XGBoosterEvalOneIter(BoosterHandle handle, int iter, DMatrixHandle dmats[], const char* evnames[],
                                 bst_ulong len, const char** out_result);
XGB_DLL int XGBoosterPredictFromDMatrix(BoosterHandle handle, DMatrixHandle dmat, char const* config,
                                        bst_ulong const** out_shape, bst_ulong* out_dim,
                                        float const** out_result);                               /* c_api.cpp:507 */
XGB_DLL int XGBoosterSaveModel(BoosterHandle handle, const char* fname);
XGB_DLL int XGBoosterLoadModel(BoosterHandle handle, const char* fname);
XGB_DLL int XGBoosterSaveModelToBuffer(BoosterHandle handle, char const* config, bst_ulong* out_len,
                                       char const** out_dptr);                                   /* c_api.cpp:521 */
XGB_DLL int XGBoosterLoadModelFromBuffer(BoosterHandle handle, const void* buf, bst_ulong len);
XGB_DLL int XGBoosterSerializeToBuffer(BoosterHandle handle, bst_ulong* out_len, const char** out_dptr);
XGB_DLL int XGBoosterUnserializeFromBuffer(BoosterHandle handle, const void* buf, bst_ulong len);
XGB_DLL int XGBoosterSaveJsonConfig(BoosterHandle handle, bst_ulong* out_len, char const** out_str);
XGB_DLL int XGBoosterLoadJsonConfig(BoosterHandle handle, char const* config);
XGB_DLL int XGBoosterBoostedRounds(BoosterHandle handle, int* out);
XGB_DLL int XGBoosterGetNumFeature(BoosterHandle handle, bst_ulong* out);
XGB_DLL int XGBoosterGetAttr(BoosterHandle handle, const char* key, const char** out, int* success);
XGB_DLL int XGBoosterSetAttr(BoosterHandle handle, const char* key, const char* value);
XGB_DLL int XGBoosterGetAttrNames(BoosterHandle handle, bst_ulong* out_len, const char*** out);
XGB_DLL int XGBoosterSetStrFeatureInfo(BoosterHandle handle, const char* field, const char** features,
                                       const bst_ulong size);
/* In-place prediction from host arrays (c_api.cpp:510-518): config as for
 * XGBoosterPredictFromDMatrix plus "missing"; the proxy argument is unused. */
XGB_DLL int XGBoosterPredictFromDense(BoosterHandle handle, char const* values, char const* config,
                                      DMatrixHandle proxy, bst_ulong const** out_shape, bst_ulong* out_dim,
                                      float const** out_result);
XGB_DLL int XGBoosterPredictFromColumnar(BoosterHandle handle, char const* values, char const* config,
                                         DMatrixHandle proxy, bst_ulong const** out_shape, bst_ulong* out_dim,
                                         float const** out_result);
XGB_DLL int XGBoosterPredictFromCSR(BoosterHandle handle, char const* indptr, char const* indices,
                                    char const* values, bst_ulong ncol, char const* config, DMatrixHandle proxy,
                                    bst_ulong const** out_shape, bst_ulong* out_dim, float const** out_result);
/* Prediction into a caller buffer of out_capacity floats (c_api.cpp:1000-1016). */
XGB_DLL int XGBoosterPredictToBuffer(BoosterHandle handle, DMatrixHandle dmat, char const* config,
                                     float* out_buffer, bst_ulong out_capacity, bst_ulong const** out_shape,
                                     bst_ulong* out_dim);
/* Feature importance over the split nodes: weight, gain, cover, total_gain,
 * total_cover (c_api.cpp:571-598). */
XGB_DLL int XGBoosterFeatureScore(BoosterHandle handle, char const* config, bst_ulong* out_n_features,
                                  char const*** out_features, bst_ulong* out_dim, bst_ulong const** out_shape,
                                  float const** out_scores);
/* Rounds [begin, end) with the given step as a new booster (model.cpp:427-440). */
XGB_DLL int XGBoosterSlice(BoosterHandle handle, int begin_layer, int end_layer, int step, BoosterHandle* out);
/* One string per tree in the text, json or dot format (model.cpp:334-425);
 * fmap: optional feature-map file ("<index> <name> <type>" lines). */
XGB_DLL int XGBoosterDumpModelEx(BoosterHandle handle, char const* fmap, int with_stats, char const* format,
                                 bst_ulong* out_len, char const*** out_dump_array);
XGB_DLL int XGBoosterDumpModel(BoosterHandle handle, char const* fmap, int with_stats, bst_ulong* out_len,
                               char const*** out_dump_array);
XGB_DLL int XGBoosterDumpModelExWithFeatures(BoosterHandle handle, int fnum, char const** fname,
                                             char const** ftype, int with_stats, char const* format,
                                             bst_ulong* out_len, char const*** out_models);
XGB_DLL int XGBoosterGetStrFeatureInfo(BoosterHandle handle, const char* field, bst_ulong* len,
                                       const char*** out_features);
/* Engine profile as JSON (device seconds per phase); counterpart of the
 * reference's XGBoosterMetalProfile (c_api.cpp:617-633). */
XGB_DLL int XGBoosterHipProfile(BoosterHandle handle, const char** out);
/* Engine extension: copy a matrix's values, labels and weights to the device
 * now (they are otherwise copied at first use) and wait for the copy. */
XGB_DLL int XGDMatrixHipUpload(DMatrixHandle handle);

/* --- single process and unsupported inputs --------------------------------
 * One process, one GPU: the communicator reports rank 0 of 1 and its
 * collectives are identities; trackers, CUDA/Arrow/DLPack/URI/buffer-
 * descriptor inputs, categorical data, external memory, separate split/leaf
 * gradients and CV-fold building return -1 naming the feature
 * (c_api.cpp:600-614 and the reference's other entry points). */
XGB_DLL int XGCommunicatorInit(char const* config);
XGB_DLL int XGCommunicatorFinalize(void);
XGB_DLL int XGCommunicatorGetRank(void);
XGB_DLL int XGCommunicatorGetWorldSize(void);
XGB_DLL int XGCommunicatorIsDistributed(void);
XGB_DLL int XGCommunicatorPrint(char const* message);
XGB_DLL int XGCommunicatorGetProcessorName(char const** name_str);
XGB_DLL int XGCommunicatorBroadcast(void* send_receive_buffer, size_t size, int root);
XGB_DLL int XGCommunicatorAllreduce(void* send_receive_buffer, size_t count, int data_type, int op);
XGB_DLL int XGCommunicatorSignalError(void);
XGB_DLL int XGTrackerCreate(char const* config, TrackerHandle* handle);
XGB_DLL int XGTrackerWorkerArgs(TrackerHandle handle, char const** args);
XGB_DLL int XGTrackerRun(TrackerHandle handle, char const* config);
XGB_DLL int XGTrackerWaitFor(TrackerHandle handle, char const* config);
XGB_DLL int XGTrackerFree(TrackerHandle handle);
XGB_DLL int XGDMatrixCreateFromCudaArrayInterface(char const* data, char const* config, DMatrixHandle* out);
XGB_DLL int XGDMatrixCreateFromCudaColumnar(char const* data, char const* config, DMatrixHandle* out);
XGB_DLL int XGProxyDMatrixSetDataCudaArrayInterface(DMatrixHandle handle, char const* data);
XGB_DLL int XGProxyDMatrixSetDataCudaColumnar(DMatrixHandle handle, char const* data);
XGB_DLL int XGBoosterPredictFromCudaArray(BoosterHandle handle, char const* values, char const* config,
                                          DMatrixHandle m, bst_ulong const** out_shape, bst_ulong* out_dim,
                                          const float** out_result);
XGB_DLL int XGBoosterPredictFromCudaColumnar(BoosterHandle handle, char const* values, char const* config,
                                             DMatrixHandle m, bst_ulong const** out_shape, bst_ulong* out_dim,
                                             const float** out_result);
XGB_DLL int XGDMatrixCreateFromArrow(void const* schema, void const* array, float missing, DMatrixHandle* out);
XGB_DLL int XGDMatrixCreateFromDLPack(void* tensor, int is_versioned, float missing, DMatrixHandle* out);
XGB_DLL int XGDMatrixCreateFromURI(char const* config, DMatrixHandle* out);
XGB_DLL int XGDMatrixCreateFromBufferDescriptor(void const* descriptor, float missing, DMatrixHandle* out);
XGB_DLL int XGDMatrixSetInfoFromBufferDescriptor(DMatrixHandle handle, char const* field, void const* descriptor);
XGB_DLL int XGBoosterPredictFromBufferDescriptor(BoosterHandle handle, void const* descriptor, char const* config,
                                                 DMatrixHandle m, bst_ulong const** out_shape, bst_ulong* out_dim,
                                                 const float** out_result);
XGB_DLL int XGExtMemQuantileDMatrixCreateFromCallback(DataIterHandle iter, DMatrixHandle proxy, DataIterHandle ref,
                                                      DataIterResetCallback* reset, XGDMatrixCallbackNext* next,
                                                      char const* config, DMatrixHandle* out);
XGB_DLL int XGBoosterTrainOneIterWithSplitGrad(BoosterHandle handle, DMatrixHandle dtrain, int iteration,
                                               char const* split_grad, char const* split_hess,
                                               char const* value_grad, char const* value_hess);
XGB_DLL int XGDMatrixBuildCVFolds(DMatrixHandle handle, int nfold, unsigned seed, int shuffle, int stratified,
                                  DMatrixHandle* out_train, DMatrixHandle* out_test);
XGB_DLL int XGDMatrixSaveBinary(DMatrixHandle handle, char const* fname, int silent);
/* No categorical features: every categories query yields a null handle. */
XGB_DLL int XGDMatrixGetCategories(DMatrixHandle handle, char const* config, CategoriesHandle* out);
XGB_DLL int XGDMatrixGetCategoriesExportToArrow(DMatrixHandle handle, char const* config, CategoriesHandle* out,
                                                char const** export_out);
XGB_DLL int XGBoosterGetCategories(BoosterHandle handle, char const* config, CategoriesHandle* out);
XGB_DLL int XGBoosterGetCategoriesExportToArrow(BoosterHandle handle, char const* config, CategoriesHandle* out,
                                                char const** export_out);
XGB_DLL int XGBCategoriesFree(CategoriesHandle handle);

#endif
