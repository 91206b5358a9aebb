"""``libortho._C_ops``: re-export of libortho_amd._C_ops (the boundary that
replaces /root/reference/torch_bind/bindings.cpp)."""
from libortho_amd._C_ops import *  # noqa: F401,F403
from libortho_amd._C_ops import forward, forward_planned, build_plan, dequant  # noqa: F401
