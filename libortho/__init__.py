"""Import-path alias so code written against the reference keeps working:
``import libortho._C_ops as _C`` (/root/reference/torch_bind/ortho_linear.py:16)
resolves to libortho_amd's operator boundary."""
