"""Loads libperegrine_hip.so and declares its C ABI (include/peregrine_hip.h).

The library is built in-tree (``peregrine_amd/build.py``). There is no CPU
fallback: if the shared object is missing, importing this module raises.
"""
from __future__ import annotations

import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libperegrine_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
        "(hipcc --offload-arch=gfx950); there is no CPU fallback")

lib = C.CDLL(LIB_PATH)

_p = C.c_void_p
_i = C.c_int
_sz = C.c_size_t
_u64p = C.POINTER(C.c_uint64)
_dp = C.POINTER(C.c_double)
_ip = C.POINTER(C.c_int)
_szp = C.POINTER(C.c_size_t)
_fp = C.POINTER(C.c_float)

# name -> (restype, argtypes); every function declared in include/peregrine_hip.h
SIGNATURES = {
    "coli_hip_init": (_i, [_ip, _i]),
    "coli_hip_shutdown": (None, []),
    "coli_hip_device_count": (_i, []),
    "coli_hip_probe_device_count": (_i, []),
    "coli_hip_device_at": (_i, [_i]),
    "coli_hip_mem_info": (_i, [_i, _szp, _szp]),
    "coli_hip_stats": (None, [_i, _szp, _szp]),
    "coli_hip_group_stats": (None, [_u64p, _u64p, _u64p, _dp, _dp, _dp]),
    "coli_hip_tensor_upload": (_i, [C.POINTER(_p), _p, _p, _i, _i, _i, _i]),
    "coli_hip_tensor_upload_grouped": (_i, [C.POINTER(_p), _p, _p, _i, _i, _i, _i, _i]),
    "coli_hip_tensor_upload_dev": (_i, [C.POINTER(_p), _p, _p, _i, _i, _i, _i, _i]),
    "coli_hip_tensor_free": (None, [_p]),
    "coli_hip_tensor_bytes": (_sz, [_p]),
    "coli_hip_tensor_device": (_i, [_p]),
    "coli_hip_tensor_update": (_i, [_p, _p, _p]),
    "coli_hip_expert_group": (_i, [_p, _p, _p, _ip, _i, _p, _p]),
    "coli_hip_expert_group_tiled": (_i, [_p, _p, _p, _ip, _i, _p, _p, _i, _i, _i, _ip]),
    "coli_hip_expert_group_reduce": (_i, [_p, _p, _p, _ip, _i, _ip, _ip, _p, _i, _p, _p]),
    "coli_hip_graph_begin": (_i, [_i]),
    "coli_hip_graph_end": (_i, [_i, C.POINTER(_p)]),
    "coli_hip_graph_launch": (_i, [_p]),
    "coli_hip_graph_free": (None, [_p]),
    "coli_hip_graph_cache_stats": (None, [_u64p, _u64p, _u64p, _u64p]),
    "coli_hip_pipe_sync": (_i, [_i]),
    "coli_hip_pipe_alloc": (_p, [_i, _sz]),
    "coli_hip_pipe_free": (None, [_i, _p]),
    "coli_hip_pipe_upload": (_i, [_i, _p, _p, _sz]),
    "coli_hip_pipe_download": (_i, [_i, _p, _p, _sz]),
    "coli_hip_event_record": (_i, [_i, _i]),
    "coli_hip_event_elapsed": (C.c_float, [_i, _i, _i]),
    "coli_hip_synth_fill": (_i, [_i, _p, _sz, _i, C.c_float, C.c_float, C.c_uint64]),
    "coli_hip_set_act_group": (_i, [_i]),
    "coli_hip_get_act_group": (_i, []),
    "coli_hip_set_arm": (_i, [_i]),
    "coli_hip_set_fused_route": (_i, [_i]),
    "coli_hip_set_fused_combine": (_i, [_i]),
    "coli_hip_set_gemv_split": (_i, [_i]),
    "coli_hip_expert_set_create": (_i, [C.POINTER(_p), _p, _p, _p, _i]),
    "coli_hip_expert_set_free": (None, [_p]),
    "coli_hip_route_softmax_topk_dev": (_i, [_i, _p, _i, _i, _i, _p, _p]),
    "coli_hip_route_sigmoid_topk_dev": (_i, [_i, _p, _p, _i, _i, _i, _i, C.c_float, C.c_float, _p, _p, _p]),
    "coli_hip_moe_forward_dev": (_i, [_p, _p, _i, _p, _p, _i, _p, _i, _i]),
    "coli_hip_moe_forward_dev_noalloc": (_i, [_p, _p, _i, _p, _p, _i, _p, _i, _i]),
    "coli_hip_moe_forward_logits_dev": (_i, [_p, _p, _i, _p, _i, _p, _p, _p, _i, _i]),
    "coli_hip_stream": (_p, [_i]),
    "coli_hip_set_profile": (_i, [_i]),
    "coli_hip_kernel_stats": (None, [_i, _u64p, _dp]),
    "coli_hip_reset_stats": (None, []),
    "coli_hip_set_debug_dots": (_i, [_p, _p]),
    "coli_hip_set_spin_limit": (_i, [_i]),
    "coli_hip_last_table": (_i, [_i, _ip, _ip, _ip, _ip, _ip, _i, _i]),
}

for _name, (_res, _args) in SIGNATURES.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args
