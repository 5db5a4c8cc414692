// Instantiations of the format templates (quant_impl.cuh) for group 1 of the formats.
#include "quant_impl.cuh"

namespace fn {

const void *qops_group1(uint32_t type) {
    switch (type) {
        case QT_BF16: return qops_of<QT_BF16>();
        case QT_Q8_0: return qops_of<QT_Q8_0>();
        case QT_IQ4_NL: return qops_of<QT_IQ4_NL>();
        default: return nullptr;
    }
}

}  // namespace fn
