// chain_f32.hip - the row chain kernel (chain_impl.h) for f32 inputs.
#include "chain_impl.h"

namespace h3 {
template int chain_launch<H3S_F32>(Ctx*, const char*, const ChainArgs&, RowPlan);
}
