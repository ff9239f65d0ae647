// Temporary: backward and calibration entry points not implemented yet.
#include "rxmet_common.h"
#include "rxmet_gru.h"
extern "C" {
int64_t rxmet_gru_backward_workspace_bytes(int32_t, int32_t, int32_t, int32_t) { return 0; }
int64_t rxmet_gru_calibrate_workspace_bytes(int32_t, int32_t, int32_t, int32_t) { return 0; }
int rxmet_gru_backward_quant(int32_t, int32_t, int32_t, int32_t, const float *, const float *, const float *, const float *, const float *, const float *, const float *, const float *, const rxmet_gru_qparams *, const uint8_t *, const uint8_t *, const uint8_t *, const uint8_t *, const uint8_t *, const uint8_t *, const uint8_t *, const uint8_t *, const uint8_t *, const uint8_t *, const uint8_t *, float *, float *, float *, float *, float *, float *, void *, void *) { rxmet::set_error("not implemented"); return -38; }
int rxmet_gru_forward_calibrate(int32_t, int32_t, int32_t, int32_t, const float *, const float *, const float *, const float *, const float *, const float *, float *, float *, float *, void *, void *) { rxmet::set_error("not implemented"); return -38; }
}
