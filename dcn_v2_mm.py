"""Import shim so code written against the reference's ``from dcn_v2_mm import
DCN`` (reference ``test.py:8``, ``train.py:12``) runs unchanged on dcnv2_amd."""
from dcnv2_amd.dcn_v2_mm import DCN, DCNv2, _DCNv2, dcn_v2_conv  # noqa: F401
