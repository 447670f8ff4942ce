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
XGB_DLL int XGBoosterGetStrFeatureInfo(BoosterHandle handle, const char* field, bst_ulong* len,
                                       const char*** out_features);
/* Engine profile as JSON (device seconds per phase); counterpart of the
 * reference's XGBoosterMetalProfile (c_api.cpp:617-633). */
XGB_DLL int XGBoosterHipProfile(BoosterHandle handle, const char** out);

#endif
