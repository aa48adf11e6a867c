"""Import shim so code written against the reference's ``from Conv2d import _C``
(reference ``dcn_v2_mm.py:12``, ``test.py:2``) runs unchanged on dcnv2_amd."""
from dcnv2_amd import _C  # noqa: F401
