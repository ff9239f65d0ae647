// Temporary: calibration entry point not implemented yet.
#include "rxmet_common.h"
#include "rxmet_gru.h"
extern "C" {
int64_t rxmet_gru_calibrate_workspace_bytes(int32_t, int32_t, int32_t, int32_t) { return 0; }
int rxmet_gru_forward_calibrate(int32_t, int32_t, int32_t, int32_t, const float *, const float *, const float *, const float *, const float *, const float *, float *, float *, float *, void *, void *) { rxmet::set_error("not implemented"); return -38; }
}
