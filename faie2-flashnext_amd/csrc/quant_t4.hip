// Instantiations of the format templates (quant_impl.cuh) for group 4 of the formats.
#include "quant_impl.cuh"

namespace fn {

const void *qops_group4(uint32_t type) {
    switch (type) {
        case QT_IQ3_S: return qops_of<QT_IQ3_S>();
        case QT_IQ3_XXS: return qops_of<QT_IQ3_XXS>();
        case QT_Q2_0: return qops_of<QT_Q2_0>();
        default: return nullptr;
    }
}

}  // namespace fn
