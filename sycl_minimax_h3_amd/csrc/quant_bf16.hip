// quant_bf16.hip - the row quantizer (quant_impl.h) for bf16 inputs.
#include "quant_impl.h"

namespace h3 {
template int quant_launch<H3S_BF16>(Ctx*, const char*, const QuantArgs&, int, RowPlan);
}
