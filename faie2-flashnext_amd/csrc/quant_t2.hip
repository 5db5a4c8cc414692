// Instantiations of the format templates (quant_impl.cuh) for group 2 of the formats.
#include "quant_impl.cuh"

namespace fn {

const void *qops_group2(uint32_t type) {
    switch (type) {
        case QT_IQ4_XS: return qops_of<QT_IQ4_XS>();
        case QT_Q4_K: return qops_of<QT_Q4_K>();
        default: return nullptr;
    }
}

}  // namespace fn
