"""The profile summarizer's kernel names: c++filt where it can, and where it
cannot (signatures holding _Float16), the nested name with its literal
template arguments, so that the committed profiles name each instantiation."""
from inferno_hip.rocpd_summary import short


def test_names_with_and_without_template_arguments():
    assert short("_ZN4ihip12k_gemv_kwideILi12ELi2ELb0ELb0ELi8EEEvPKhS2_PKfPfiiS4_fS4_i") == \
        "k_gemv_kwide<12, 2, false, false, 8>"
    # _Float16 parameters: the fallback parser
    assert short("_ZN4ihip13k_prefill_q4kILb0EEEvPKhPKDF16_PKiPfS6_iiiiii") == "k_prefill_q4k<false>"
    assert short("_ZN4ihip13k_prefill_q4kILb1EEEvPKhPKDF16_PKiPfS6_iiiiii") == "k_prefill_q4k<true>"
    assert short("_ZN4ihip10k_x_to_f16EPKfPDF16_Pii") == "k_x_to_f16"
    assert short("_ZN4ihip17k_prefill_q4k_f32EPKhPKfPfiiii") == "k_prefill_q4k_f32"
    assert short("__amd_rocclr_copyBuffer") == "__amd_rocclr_copyBuffer"
