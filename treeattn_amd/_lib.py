"""ctypes binding of libtreeattn.so (the C ABI declared in include/treeattn.h).

The library is loaded after torch so it binds to the HIP runtime torch already loaded.  Every call passes
device pointers, element strides and torch's current HIP stream; a non-zero status raises RuntimeError
with the library's message.  There is no fallback: a missing library, a non-GPU tensor or an unsupported
device raises.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, 'libtreeattn.so')

F32, F16, BF16 = 0, 1, 2
_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

c_i32, c_i64, c_f32, c_vp = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p
_P = ctypes.POINTER

MAX_TREE_LEVELS = 32


class KvPages(ctypes.Structure):
    """ta_kv_pages"""
    _fields_ = [('table', c_vp), ('sb', c_i64), ('sh', c_i64), ('page_stride', c_i64), ('num_pages', c_i64),
                ('block_log2', c_i32)]


class LeafStoreOut(ctypes.Structure):
    """ta_leaf_store_out (include/treeattn.h)."""
    _fields_ = [('leaf', c_vp), ('score', c_vp), ('ok', c_vp), ('sb', c_i64), ('sh', c_i64), ('st', c_i64),
                ('Tst', c_i32), ('n', c_i32)]


class BudgetHeadIn(ctypes.Structure):
    """ta_budget_head_in (include/treeattn.h)."""
    _fields_ = [('w1t', c_vp), ('b1', c_vp), ('w2', c_vp), ('b2', c_vp), ('classes', c_vp), ('hid', c_i32),
                ('ncls', c_i32), ('ksum', c_vp), ('k', c_vp), ('ksb', c_i64), ('ksh', c_i64), ('lhat', c_vp)]


class StepLayer(ctypes.Structure):
    """ta_step_layer"""
    _fields_ = [('ln1', c_vp), ('c_attn', c_vp), ('c_proj', c_vp), ('ln2', c_vp), ('c_fc', c_vp), ('c_mlp', c_vp),
                ('k_cache', c_vp), ('v_cache', c_vp), ('c_sb', c_i64), ('c_sh', c_i64), ('c_st', c_i64),
                ('levels', c_vp * MAX_TREE_LEVELS), ('lv_sb', c_i64 * MAX_TREE_LEVELS),
                ('lv_sh', c_i64 * MAX_TREE_LEVELS)]


class StepModel(ctypes.Structure):
    """ta_step_model"""
    _fields_ = [('n_layer', c_i32), ('n_head', c_i32), ('head_dim', c_i32), ('n_embd', c_i32), ('n_ff', c_i32),
                ('vocab', c_i32), ('n_pos', c_i32), ('batch', c_i32), ('tcap', c_i32), ('leaf', c_i32),
                ('arity', c_i32), ('n_levels', c_i32), ('wmax', c_i32), ('n_tree', c_i32), ('local', c_i32),
                ('mlp_splits', c_i32), ('ln_eps', c_f32), ('wte', c_vp), ('ld_wte', c_i64), ('wpe', c_vp),
                ('ld_wpe', c_i64), ('ln_f', c_vp), ('layers', ctypes.POINTER(StepLayer))]


class StepLaunch(ctypes.Structure):
    """ta_step_launch"""
    _fields_ = [('grid', c_i32), ('lds_bytes', c_i32), ('n_tasks', c_i32), ('head_dim', c_i32)]


# name -> (restype, argtypes); mirrors include/treeattn.h
SIGNATURES = {
    'ta_abi_version': (c_i32, []),
    'ta_last_error': (ctypes.c_char_p, []),
    'ta_device_supported': (c_i32, []),
    'ta_level_sums_workspace_size': (c_i64, [c_i32, c_i32, c_i32, c_i32]),
    'ta_level_sums': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
                              _P(c_vp), _P(c_i64), _P(c_i64), _P(ctypes.c_int32), c_vp, c_i64, c_vp]),
    'ta_tree_descend': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_vp, c_i64,
                                c_i32, _P(c_vp), _P(c_i64), _P(c_i64), c_i32, c_i32, c_i32, c_i32, c_i32,
                                c_vp, c_vp, c_vp, c_vp]),
    'ta_tree_descend_store': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_vp, c_i64,
                                      c_i32, _P(c_vp), _P(c_i64), _P(c_i64), c_i32, c_i32, c_i32, c_i32, c_i32,
                                      c_vp, c_vp, c_vp, _P(LeafStoreOut), c_vp]),
    'ta_tree_descend_append': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i32, c_i32, c_i32, c_vp, c_i32, _P(c_vp),
                                       _P(c_i64), _P(c_i64), c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp, c_vp,
                                       c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64, c_i64,
                                       c_i32, _P(KvPages), c_vp]),
    'ta_tree_descend_append_ex': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i32, c_i32, c_i32, c_vp, c_i32, _P(c_vp),
                                          _P(c_i64), _P(c_i64), c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp,
                                          c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64,
                                          c_i64, c_i32, _P(KvPages), _P(c_vp), _P(c_i64), _P(c_i64), _P(c_vp),
                                          _P(c_vp), c_f32, _P(LeafStoreOut), c_vp]),
    'ta_seg_attend': (c_i32, [c_vp, c_vp, c_vp, c_i32, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i32, c_i32,
                              c_i32, c_vp, c_i32, _P(c_vp), _P(c_i64), _P(c_i64), c_i32, c_i32, c_i32, c_i32, c_i32,
                              c_vp, c_vp, c_i64, c_i64, c_i64, c_i32, c_vp, c_i32, c_f32, c_vp, c_vp, c_vp, c_vp,
                              c_i64, c_i64, c_vp, _P(KvPages), c_vp]),
    'ta_gather_dot': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_vp, c_i32, c_i64, c_i64, c_i64, c_vp,
                              c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_f32, c_vp, c_vp]),
    'ta_gather_dot_blocks': (c_i32, [c_vp, c_vp, c_i32, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp,
                                     c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_f32, c_vp, c_vp]),
    'ta_assemble_candidates': (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
                                       c_i32, c_vp, c_vp, c_vp]),
    'ta_sparse_attn_fwd': (c_i32, [c_vp, c_vp, c_vp, c_i32, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                   c_i64, c_i64, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_f32, c_vp,
                                   c_vp, _P(KvPages), c_vp]),
    'ta_sparse_attn_bwd': (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_i32] + [c_i64] * 15 + [c_vp, c_vp] + [c_i32] * 6
                           + [c_f32, c_vp, c_vp, c_vp, c_vp, c_i32, c_vp]),
    'ta_sparse_attn_bwd_workspace_size': (c_i64, [c_i32, c_i32, c_i32, c_i32]),
    'ta_seg_attn_workspace_size': (c_i64, [c_i32, c_i32, c_i32, c_i32, c_i32]),
    'ta_seg_attn_fwd': (c_i32, [c_vp, c_vp, c_vp, c_i32, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_i64, c_vp, c_vp, c_vp, c_i32,
                                c_i32, c_i32, c_f32, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_i32, c_vp, c_i64,
                                _P(KvPages), c_vp]),
    'ta_seg_attn_nb_fwd': (c_i32, [c_vp, c_vp, c_vp, c_i32, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                   c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_i64, c_vp, c_vp, c_vp,
                                   c_i32, c_i32, c_i32, c_f32, c_vp, c_vp, c_i32, c_vp, c_i64, c_i64, c_i64, c_vp,
                                   c_vp, c_i32, c_vp, c_i64, _P(KvPages), c_vp]),
    'ta_seg_attn_fwd_noalloc': (c_i32, [c_vp, c_vp, c_vp, c_i32, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                        c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_i64, c_vp, c_vp,
                                        c_vp, c_i32, c_i32, c_i32, c_f32, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp,
                                        c_i32, _P(KvPages), c_vp]),
    'ta_kv_append': (c_i32, [c_vp, c_vp, c_i32, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64, c_i64,
                             c_i32, c_i32, c_i32, c_i32, c_vp, c_i32, _P(c_vp), _P(c_i64), _P(c_i64), c_i32,
                             c_i32, _P(KvPages), c_vp]),
    'ta_argmax_rows': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_vp, c_vp]),
    'ta_embed': (c_i32, [c_vp, c_vp, c_i32, c_vp, c_i64, c_vp, c_i64, c_i32, c_i32, c_i32, c_i64, c_i64, c_vp,
                         c_i64, c_vp, c_vp, c_f32, c_vp, c_i64, c_vp]),
    'ta_rowmm_workspace_size': (c_i64, [c_i32, c_i32, c_i32, c_i32]),
    'ta_rowmm': (c_i32, [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_f32, c_i32, c_i32, c_i32, c_i32,
                         c_i32, c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp]),
    'ta_rowmm_ex': (c_i32, [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_f32, c_i32, c_i32, c_i32,
                            c_i32, c_i32, c_i32, c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp]),
    'ta_mfma_peak': (c_i32, [c_i32, c_i32, c_vp, c_vp]),
    'ta_forest_build': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
                                c_f32, c_f32, c_vp, _P(c_vp), _P(c_vp), _P(c_i64), _P(c_i64), c_vp]),
    'ta_forest_descend': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, _P(c_vp),
                                  _P(c_i64), _P(c_i64), c_vp, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i32,
                                  c_vp, c_vp]),
    'ta_forest_shape': (c_i32, [c_i32, c_i32, c_i32, _P(c_i32), _P(c_i32), _P(c_i32)]),
    'ta_lanetree_workspace_size': (c_i32, [c_i32, c_i32, c_i32, c_i32, c_i32, _P(c_i64)]),
    'ta_lanetree_build': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp,
                                  c_i64, c_vp]),
    'ta_lanetree_walk': (c_i32, [c_vp, c_vp, c_i32, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32,
                                 c_i32, c_i32, c_vp, c_i32, c_i32, c_i32, c_f32, c_i32, c_i32, c_i32, c_vp, c_i64,
                                 c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    'ta_level_log_sums': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
                                  _P(c_vp), _P(c_i64), _P(c_i64), _P(c_i32), c_vp, c_i64, c_vp]),
    'ta_gate_levels': (c_i32, [c_i32, c_i32, c_i32, c_i32, _P(c_vp), _P(c_vp), _P(c_vp), _P(c_i64), _P(c_i64),
                               _P(c_i32), _P(c_i64), c_f32, c_vp]),
    'ta_gate_append': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_vp, c_i32, _P(c_vp),
                               _P(c_vp), _P(c_vp), _P(c_i64), _P(c_i64), _P(c_i32), c_i32, c_f32, _P(KvPages),
                               c_vp]),
    'ta_neighbor_pass': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_i64, c_vp, c_i64, c_i64, c_i32, c_vp, c_vp, c_vp,
                                 c_i64, c_i64, c_i64, c_i32, c_vp, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
                                 c_i32, c_i32, c_f32, c_i32, c_f32, c_vp, c_i32, c_vp, c_vp, c_vp, c_vp, c_vp]),
    'ta_budget_head': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp]),
    'ta_neighbor_pass_head': (c_i32, [c_vp, c_i32, c_i64, c_i64, c_vp, c_i64, c_i64, c_i32, c_vp, c_vp, c_vp, c_i64,
                                      c_i64, c_i64, c_i32, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
                                      c_f32, c_i32, c_f32, c_i32, _P(BudgetHeadIn), c_vp, c_vp, c_vp, c_vp,
                                      c_vp]),
    'ta_leaf_store': (c_i32, [c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64,
                              c_i32, c_vp]),
    'ta_logits_workspace_size': (c_i64, [c_i32, c_i32]),
    'ta_logits': (c_i32, [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_f32, c_i32, c_i32, c_i32, c_vp, c_vp, c_i64,
                          c_vp]),
    'ta_bf16_from_f32': (c_i32, [c_vp, c_vp, c_i64, c_vp]),
    'ta_rowvec_f32': (c_i32, [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_f32, c_i32, c_i32, c_i32,
                               c_i32, c_vp]),
    'ta_rowvec_bf16': (c_i32, [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_f32, c_i32, c_i32, c_i32,
                                c_i32, c_vp]),
    'ta_decode_step_workspace_size': (c_i64, [_P(StepModel)]),
    'ta_decode_step_prepare': (c_i32, [_P(StepModel), c_vp, c_i64, _P(StepLaunch), c_vp]),
    'ta_decode_step': (c_i32, [_P(StepLaunch), c_vp, c_vp, c_vp, c_vp, c_i32, c_vp, c_i64, c_vp, c_vp, c_vp]),
    'ta_decode_step_error': (c_i32, [c_vp, _P(c_i32), c_vp]),
}

_lib = None


def lib():
    """Load (once) and return the library.  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError('treeattn_amd: %s is missing; build it with `python -m treeattn_amd.build`'
                               % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc, name):
    if rc != 0:
        msg = lib().ta_last_error().decode(errors='replace')
        raise RuntimeError('treeattn_amd: %s failed (status %d): %s' % (name, rc, msg))


def call(name, *args):
    check(getattr(lib(), name)(*args), name)


def dtype_code(t):
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError('treeattn_amd: unsupported dtype %s' % t.dtype) from None


_checked_devices = set()


def require_gpu(*tensors):
    """Every tensor must live on a supported GPU; the first use of a device checks it is a gfx950."""
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError('treeattn_amd: tensors must be on the GPU (got %s); there is no CPU path'
                               % t.device)
        dev = t.device.index if t.device.index is not None else torch.cuda.current_device()
        if dev not in _checked_devices:
            with torch.cuda.device(dev):
                if lib().ta_device_supported() != 1:
                    raise RuntimeError('treeattn_amd: device %d is not a gfx950 (MI355X)' % dev)
            _checked_devices.add(dev)


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def rows3(t):
    """Strides (b, h, n) in elements of a (B, H, N, D) tensor whose last dimension is contiguous."""
    if t.stride(-1) != 1:
        raise ValueError('treeattn_amd: last dimension must be contiguous')
    return t.stride(0), t.stride(1), t.stride(2)


def ptr_array(tensors):
    return (c_vp * max(1, len(tensors)))(*[t.data_ptr() for t in tensors])


def i64_array(vals):
    return (c_i64 * max(1, len(vals)))(*vals)


def i32_array(vals):
    return (ctypes.c_int32 * max(1, len(vals)))(*vals)
