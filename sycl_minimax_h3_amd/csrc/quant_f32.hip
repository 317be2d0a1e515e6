// quant_f32.hip - the row quantizer (quant_impl.h) for f32 inputs.
#include "quant_impl.h"

namespace h3 {
template int quant_launch<H3S_F32>(Ctx*, const char*, const QuantArgs&, int, RowPlan);
}
