// chain_f16.hip - the row chain kernel (chain_impl.h) for f16 inputs.
#include "chain_impl.h"

namespace h3 {
template int chain_launch<H3S_F16>(Ctx*, const char*, const ChainArgs&, RowPlan);
}
