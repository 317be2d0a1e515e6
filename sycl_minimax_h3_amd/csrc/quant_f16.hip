// quant_f16.hip - the row quantizer (quant_impl.h) for f16 inputs.
#include "quant_impl.h"

namespace h3 {
template int quant_launch<H3S_F16>(Ctx*, const char*, const QuantArgs&, int, RowPlan);
}
