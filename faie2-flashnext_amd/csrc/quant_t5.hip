// Instantiations of the format templates (quant_impl.cuh) for group 5 of the formats.
#include "quant_impl.cuh"

namespace fn {

const void *qops_group5(uint32_t type) {
    switch (type) {
        case QT_IQ2_XXS: return qops_of<QT_IQ2_XXS>();
        case QT_IQ2_XS: return qops_of<QT_IQ2_XS>();
        case QT_IQ2_S: return qops_of<QT_IQ2_S>();
        default: return nullptr;
    }
}

}  // namespace fn
