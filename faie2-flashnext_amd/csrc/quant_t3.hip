// Instantiations of the format templates (quant_impl.cuh) for group 3 of the formats.
#include "quant_impl.cuh"

namespace fn {

const void *qops_group3(uint32_t type) {
    switch (type) {
        case QT_Q5_K: return qops_of<QT_Q5_K>();
        case QT_Q6_K: return qops_of<QT_Q6_K>();
        default: return nullptr;
    }
}

}  // namespace fn
