"""ctypes binding of libcheddar_amd.so (include/cheddar_amd.h).

Device buffers are torch tensors on the HIP device (torch is only the
allocator and stream provider here). Every function raises ChdError with
the library's message on a non-zero status. Importing this module fails
loudly if the HIP library has not been built.
"""
import ctypes
import os
import weakref

import numpy as np

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG, "lib", "libcheddar_amd.so")
LOG_N = 16
N = 1 << LOG_N


class ChdError(RuntimeError):
    pass


if not os.path.exists(LIB_PATH):
    raise ImportError("libcheddar_amd.so is not built: run "
                      "python cheddar-fhe_amd/build.py")

_c_u32p = ctypes.POINTER(ctypes.c_uint32)
_c_i32p = ctypes.POINTER(ctypes.c_int32)
_vp = ctypes.c_void_p
_i = ctypes.c_int
_pp = ctypes.POINTER(ctypes.c_void_p)
_ip = ctypes.POINTER(ctypes.c_int)
_dp = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")

lib = ctypes.CDLL(LIB_PATH)
_SIGS = {
    "chd_last_error": (ctypes.c_char_p, []),
    "chd_version": (ctypes.c_char_p, []),
    "chd_ntt_plan_create": (_i, [_pp, _i, _c_u32p, _i]),
    "chd_ntt_plan_destroy": (None, [_vp]),
    "chd_ntt_plan_tables": (_vp, [_vp]),
    "chd_ntt_forward": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "chd_ntt_inverse": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "chd_ntt_inverse_single_pass": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "chd_ntt_forward_two_pass": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "chd_bconv_plan_create": (_i, [_pp, _i, _c_u32p, _i, _c_u32p, _i]),
    "chd_bconv_plan_destroy": (None, [_vp]),
    "chd_bconv_plan_constants": (_i, [_vp, _c_u32p, _c_i32p]),
    "chd_bconv_apply": (_i, [_vp, _vp, _vp, _vp]),
    "chd_param_create": (_i, [_pp, _i, ctypes.c_double, _i,
                              ctypes.POINTER(ctypes.c_int), _i, _c_u32p, _i,
                              _c_u32p, _i, _c_u32p, _i]),
    "chd_param_create_json": (_i, [_pp, ctypes.c_char_p]),
    "chd_param_destroy": (None, [_vp]),
    "chd_param_num_q": (_i, [_vp, _i]),
    "chd_param_alpha": (_i, [_vp]),
    "chd_param_max_level": (_i, [_vp]),
    "chd_param_evk_limbs": (_i, [_vp]),
    "chd_context_create": (_i, [_pp, _vp]),
    "chd_context_destroy": (None, [_vp]),
    "chd_context_beta": (_i, [_vp, _i]),
    "chd_tensor": (_i, [_vp, _i] + [_vp] * 7 + [_vp]),
    "chd_mod_up": (_i, [_vp, _i, _pp, _vp, _vp]),
    "chd_mod_down": (_i, [_vp, _i, _vp, _vp, _vp]),
    "chd_rescale_poly": (_i, [_vp, _i, _vp, _vp, _vp]),
    "chd_mod_down_and_rescale": (_i, [_vp, _i, _vp, _vp, _vp]),
    "chd_hmult": (_i, [_vp, _i] + [_vp] * 6 + [_pp, _pp, _i, _i, _vp]),
    "chd_hmult_noalloc": (_i, [_vp, _i] + [_vp] * 6 + [_pp, _pp, _i, _i,
                                                     _vp]),
    "chd_rescale": (_i, [_vp, _i] + [_vp] * 4 + [_vp]),
    "chd_mult_key": (_i, [_vp, _i] + [_vp] * 4 + [_pp, _pp, _i, _vp]),
    "chd_mult_key_no_mod_down": (_i, [_vp, _i] + [_vp] * 5 + [_pp, _pp, _i,
                                                             _vp]),
    "chd_mult_key_no_mod_down_mod_up": (_i, [_vp, _i, _vp, _vp, _pp, _pp, _pp,
                                             _i, _vp]),
    "chd_hrot": (_i, [_vp, _i] + [_vp] * 4 + [_pp, _pp, _i, _i, _i, _vp]),
    "chd_permute": (_i, [_vp, _i] + [_vp] * 4 + [_i, _vp]),
    "chd_hoist_baby_steps": (_i, [_vp, _i, _vp, _vp, _i, _ip, _pp, _pp, _i,
                                  _ip, _pp, _pp, _i, _vp]),
    "chd_hoist_evaluate": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _i, _ip, _i, _ip,
                                _pp, _i, _ip, _pp, _pp, _i, _vp]),
    "chd_hoist_create": (_i, [_pp, _vp, _i, _i, _ip, _i, _ip, _pp, _vp]),
    "chd_hoist_destroy": (None, [_vp]),
    "chd_hoist_run_min_ks": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _ip, _pp, _pp,
                                  _i, _vp]),
    "chd_hoist_required_rotations": (_i, [_vp, _i, _ip, _i]),
    "chd_linear_transform_create": (_i, [_pp, _vp, _i, ctypes.c_double, _i,
                                         _i, _ip, _pp, _pp, _i, _i, _i, _i,
                                         _vp]),
    "chd_hoist_create_from_messages": (_i, [_pp, _vp, _i, ctypes.c_double,
                                            _i, _ip, _i, _ip, _pp, _pp, _ip,
                                            _i, _vp]),
    "chd_elementwise": (_i, [_vp, _i, _i, _i, _i, _pp, _pp, _pp, _vp, _vp]),
    "chd_encode": (_i, [_vp, _i, _i, ctypes.c_double, _dp, _dp, _i, _vp,
                        _vp]),
    "chd_encode_constant": (_i, [_vp, _i, _i, ctypes.c_double,
                                 ctypes.c_double, _vp, _vp]),
    "chd_decode": (_i, [_vp, _i, ctypes.c_double, _i, _vp, _dp, _dp, _vp]),
    "chd_encode_coefficients": (_i, [_vp, _i, _i, ctypes.c_double, _dp, _dp,
                                     _i, _u32p]),
    "chd_hoist_run": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _ip, _pp, _pp, _i,
                           _vp]),
}
for _name, (_res, _args) in _SIGS.items():
    _f = getattr(lib, _name)
    _f.restype = _res
    _f.argtypes = _args


def _split(msg):
    m = np.asarray(msg, np.complex128).reshape(-1)
    return (np.ascontiguousarray(m.real, np.float64),
            np.ascontiguousarray(m.imag, np.float64))


def _check(status):
    if status != 0:
        raise ChdError(lib.chd_last_error().decode())


def _u32_array(vals):
    return (ctypes.c_uint32 * len(vals))(*[int(v) for v in vals])


def ptr(t):
    """device pointer of a torch tensor (or None)"""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def ptr_array(ts):
    """device pointers of torch tensors (None gives NULL)"""
    return (ctypes.c_void_p * len(ts))(
        *[None if t is None else t.data_ptr() for t in ts])


def _own(obj, h, destroy):
    """obj takes ownership of handle h: destroy(h) runs once, when obj is
    collected or at interpreter exit (bound now, so it never depends on
    module globals that exit may already have cleared)"""
    obj.h = h
    obj._finalizer = weakref.finalize(obj, destroy, h)


def current_stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class NttPlan:
    """standalone NTT over an explicit prime chain (configs 1-2)"""

    def __init__(self, primes, log_n=LOG_N):
        self.primes = [int(p) for p in primes]
        h = ctypes.c_void_p()
        _check(lib.chd_ntt_plan_create(ctypes.byref(h), log_n,
                                       _u32_array(self.primes),
                                       len(self.primes)))
        _own(self, h, lib.chd_ntt_plan_destroy)


    def forward(self, dst, src, num_limbs, num_polys=1, mont_conv=False,
                stream=None, two_pass=False):
        """two_pass: always the two-pass kernels (the same results; for
        throughput over several streams, where they share the GPU better)"""
        fn = lib.chd_ntt_forward_two_pass if two_pass else lib.chd_ntt_forward
        _check(fn(self.h, ptr(dst), ptr(src), num_limbs, num_polys,
                  int(bool(mont_conv)),
                  stream if stream is not None else current_stream()))

    def inverse(self, dst, src, num_limbs, num_polys=1, mont_conv=True,
                stream=None, single_pass=False):
        """single_pass: the one-pass kernel over residue classes (dst apart
        from src; the default two passes are faster)"""
        fn = (lib.chd_ntt_inverse_single_pass if single_pass
              else lib.chd_ntt_inverse)
        _check(fn(self.h, ptr(dst), ptr(src), num_limbs, num_polys,
                  int(bool(mont_conv)),
                  stream if stream is not None else current_stream()))


class BconvPlan:
    """standalone BConv src primes -> dst primes (config 3)"""

    def __init__(self, src_primes, dst_primes, log_n=LOG_N):
        self.src = [int(p) for p in src_primes]
        self.dst = [int(p) for p in dst_primes]
        h = ctypes.c_void_p()
        _check(lib.chd_bconv_plan_create(ctypes.byref(h), log_n,
                                         _u32_array(self.src), len(self.src),
                                         _u32_array(self.dst), len(self.dst)))
        _own(self, h, lib.chd_bconv_plan_destroy)


    def constants(self):
        import numpy as np
        c1 = np.zeros(len(self.src), np.uint32)
        c2 = np.zeros(len(self.src) * len(self.dst), np.int32)
        _check(lib.chd_bconv_plan_constants(
            self.h, c1.ctypes.data_as(_c_u32p), c2.ctypes.data_as(_c_i32p)))
        return c1, c2.reshape(len(self.dst), len(self.src))

    def apply(self, dst, src_centred, stream=None):
        _check(lib.chd_bconv_apply(self.h, ptr(dst), ptr(src_centred),
                                   stream if stream is not None else
                                   current_stream()))


class Param:
    def __init__(self, main_primes, aux_primes, level_config,
                 default_encryption_level=None, base_scale=float(1 << 30),
                 log_n=LOG_N):
        lc = [int(v) for pair in level_config for v in pair]
        dl = (len(level_config) - 1 if default_encryption_level is None
              else default_encryption_level)
        h = ctypes.c_void_p()
        _check(lib.chd_param_create(
            ctypes.byref(h), log_n, base_scale, dl,
            (ctypes.c_int * len(lc))(*lc), len(level_config),
            _u32_array(main_primes), len(main_primes),
            _u32_array(aux_primes), len(aux_primes), None, 0))
        _own(self, h, lib.chd_param_destroy)
        self.main = [int(p) for p in main_primes]
        self.aux = [int(p) for p in aux_primes]
        self.alpha = lib.chd_param_alpha(h)
        self.max_level = lib.chd_param_max_level(h)
        self.evk_limbs = lib.chd_param_evk_limbs(h)

    @classmethod
    def from_json(cls, text):
        """a parameter set in the reference's JSON layout (parameters/*.json)"""
        import json
        self = cls.__new__(cls)
        h = ctypes.c_void_p()
        _check(lib.chd_param_create_json(ctypes.byref(h), text.encode()))
        _own(self, h, lib.chd_param_destroy)
        d = json.loads(text)
        self.main = [int(p) for p in d["main_primes"]]
        self.ter = [int(p) for p in d.get("terminal_primes", [])]
        self.aux = [int(p) for p in d["auxiliary_primes"]]
        self.level_config = [tuple(c) for c in d["level_config"]]
        self.alpha = lib.chd_param_alpha(h)
        self.max_level = lib.chd_param_max_level(h)
        self.evk_limbs = lib.chd_param_evk_limbs(h)
        return self

    def num_q(self, level):
        return lib.chd_param_num_q(self.h, level)

    def encode_coefficients(self, level, num_aux, scale, msg, log_n=LOG_N,
                            out=None):
        """host half of the encoder: (residues [limbs][N] before the NTT,
        padded slot count); out: an optional uint32 buffer of that size"""
        re, im = _split(msg)
        words = (self.num_q(level) + num_aux) << log_n
        if out is None:
            out = np.zeros(words, np.uint32)
        elif (out.dtype != np.uint32 or out.size != words or
              not out.flags["C_CONTIGUOUS"]):
            raise ValueError("encode_coefficients: out must be a contiguous "
                             "uint32 array of %d words" % words)
        out = out.reshape(-1)
        slots = lib.chd_encode_coefficients(self.h, level, num_aux, scale, re,
                                            im, re.size, out)
        if slots < 0:
            _check(slots)
        return out.reshape(-1, 1 << log_n), slots



class Context:
    def __init__(self, param):
        self.param = param
        h = ctypes.c_void_p()
        _check(lib.chd_context_create(ctypes.byref(h), param.h))
        _own(self, h, lib.chd_context_destroy)


    def beta(self, level):
        return lib.chd_context_beta(self.h, level)

    def _s(self, stream):
        return stream if stream is not None else current_stream()

    def tensor(self, level, res, a, b, stream=None):
        _check(lib.chd_tensor(self.h, level, *[ptr(t) for t in res],
                              *[ptr(t) for t in a], *[ptr(t) for t in b],
                              self._s(stream)))

    def mod_up(self, level, dst_list, src, stream=None):
        _check(lib.chd_mod_up(self.h, level, ptr_array(dst_list), ptr(src),
                              self._s(stream)))

    def mod_down(self, level, dst, src, stream=None):
        _check(lib.chd_mod_down(self.h, level, ptr(dst), ptr(src),
                                self._s(stream)))

    def rescale_poly(self, level, dst, src, stream=None):
        _check(lib.chd_rescale_poly(self.h, level, ptr(dst), ptr(src),
                                    self._s(stream)))

    def mod_down_and_rescale(self, level, dst, src, stream=None):
        _check(lib.chd_mod_down_and_rescale(self.h, level, ptr(dst), ptr(src),
                                            self._s(stream)))

    def hmult(self, level, res, a, b, evk_b, evk_a, rescale=True,
              stream=None):
        _check(lib.chd_hmult(self.h, level, ptr(res[0]), ptr(res[1]),
                             ptr(a[0]), ptr(a[1]), ptr(b[0]), ptr(b[1]),
                             ptr_array(evk_b), ptr_array(evk_a), len(evk_b),
                             int(bool(rescale)), self._s(stream)))

    def hmult_noalloc(self, level, res, a, b, evk_b, evk_a, rescale=True,
                      stream=None):
        """hmult with its temporaries in the library's static device array
        (no device allocation)"""
        _check(lib.chd_hmult_noalloc(self.h, level, ptr(res[0]), ptr(res[1]),
                                     ptr(a[0]), ptr(a[1]), ptr(b[0]),
                                     ptr(b[1]), ptr_array(evk_b),
                                     ptr_array(evk_a), len(evk_b),
                                     int(bool(rescale)), self._s(stream)))

    def rescale(self, level, res, a, stream=None):
        _check(lib.chd_rescale(self.h, level, ptr(res[0]), ptr(res[1]),
                               ptr(a[0]), ptr(a[1]), self._s(stream)))

    def mult_key(self, level, res, a, evk_b, evk_a, stream=None):
        _check(lib.chd_mult_key(self.h, level, ptr(res[0]), ptr(res[1]),
                                ptr(a[0]), ptr(a[1]), ptr_array(evk_b),
                                ptr_array(evk_a), len(evk_b),
                                self._s(stream)))

    def mult_key_no_mod_down(self, level, acc, a, evk_b, evk_a, stream=None):
        """Context::MultKeyNoModDown(accum, a, key): acc = (acc_b, acc_a) of
        num_q + alpha limbs; a = (bx, ax) or (bx, ax, rx)"""
        rx = a[2] if len(a) > 2 else None
        _check(lib.chd_mult_key_no_mod_down(
            self.h, level, ptr(acc[0]), ptr(acc[1]), ptr(a[0]), ptr(a[1]),
            ptr(rx), ptr_array(evk_b), ptr_array(evk_a), len(evk_b),
            self._s(stream)))

    def mult_key_no_mod_down_mod_up(self, level, acc, a_modup, evk_b, evk_a,
                                    stream=None):
        """Context::MultKeyNoModDown(accum, a_modup, a_orig, key): a_modup is
        the list mod_up wrote (None for groups holding no limb of level)"""
        _check(lib.chd_mult_key_no_mod_down_mod_up(
            self.h, level, ptr(acc[0]), ptr(acc[1]), ptr_array(a_modup),
            ptr_array(evk_b), ptr_array(evk_a), len(evk_b), self._s(stream)))

    def hrot(self, level, res, a, evk_b, evk_a, rot, num_slots=N // 2,
             stream=None):
        _check(lib.chd_hrot(self.h, level, ptr(res[0]), ptr(res[1]),
                            ptr(a[0]), ptr(a[1]), ptr_array(evk_b),
                            ptr_array(evk_a), len(evk_b), rot, num_slots,
                            self._s(stream)))

    @staticmethod
    def _keys(keys):
        """{rot: (bx groups, ax groups)} -> key_rot, key_bx, key_ax, beta"""
        rots = sorted(keys)
        beta = len(keys[rots[0]][0]) if rots else 1
        kb = [t for r in rots for t in keys[r][0]]
        ka = [t for r in rots for t in keys[r][1]]
        return ((ctypes.c_int * max(1, len(rots)))(*rots), ptr_array(kb),
                ptr_array(ka), len(rots), beta)

    def hoist_baby_steps(self, level, ct, rots, dst, keys, stream=None):
        """dst[i] = (bx, ax) tensors of num_q(level) + alpha limbs"""
        kr, kb, ka, nk, beta = self._keys(keys)
        _check(lib.chd_hoist_baby_steps(
            self.h, level, ptr(ct[0]), ptr(ct[1]), len(rots),
            (ctypes.c_int * len(rots))(*rots), ptr_array([d[0] for d in dst]),
            ptr_array([d[1] for d in dst]), nk, kr, kb, ka, beta,
            self._s(stream)))

    def hoist_evaluate(self, level, res, ct, gs, bs, pts, keys, stream=None):
        """pts: {(g, b): tensor of num_q(level) + alpha limbs}"""
        kr, kb, ka, nk, beta = self._keys(keys)
        parr = (ctypes.c_void_p * (len(gs) * len(bs)))(*[
            pts[(g, b)].data_ptr() if (g, b) in pts else None
            for g in gs for b in bs])
        _check(lib.chd_hoist_evaluate(
            self.h, level, ptr(res[0]), ptr(res[1]), ptr(ct[0]), ptr(ct[1]),
            len(gs), (ctypes.c_int * len(gs))(*gs), len(bs),
            (ctypes.c_int * len(bs))(*bs), parr, nk, kr, kb, ka, beta,
            self._s(stream)))

    EW_OPS = {"add": 0, "sub": 1, "neg": 2, "mult": 3, "pmult": 4,
              "add_const": 5, "sub_const": 6, "sub_opp_const": 7,
              "mult_const": 8, "mult_i": 9, "copy": 10}

    def elementwise(self, level, num_aux, op, dst, a, b=None, cst=None,
                    stream=None):
        """ElementWiseHandler op on lists of polynomials (device tensors)"""
        _check(lib.chd_elementwise(
            self.h, level, num_aux, self.EW_OPS[op], len(dst),
            ptr_array(dst), ptr_array(a),
            ptr_array(b) if b is not None else None, ptr(cst),
            self._s(stream)))

    def encode(self, level, num_aux, scale, msg, dst, stream=None):
        """message (complex array) -> plaintext limbs in dst (device);
        returns the padded slot count"""
        re, im = _split(msg)
        slots = lib.chd_encode(self.h, level, num_aux, scale, re, im, re.size,
                               ptr(dst), self._s(stream))
        if slots < 0:
            _check(slots)
        return slots

    def encode_constant(self, level, num_aux, scale, number, dst,
                        stream=None):
        _check(lib.chd_encode_constant(self.h, level, num_aux, scale,
                                       float(number), ptr(dst),
                                       self._s(stream)))

    def decode(self, level, scale, num_slots, src, stream=None):
        re = np.zeros(num_slots, np.float64)
        im = np.zeros(num_slots, np.float64)
        _check(lib.chd_decode(self.h, level, scale, num_slots, ptr(src), re,
                              im, self._s(stream)))
        return re + 1j * im

    def permute(self, level, res, a, rot, stream=None):
        _check(lib.chd_permute(self.h, level, ptr(res[0]), ptr(res[1]),
                               ptr(a[0]), ptr(a[1]), rot, self._s(stream)))


class Hoist:
    """HoistHandler built once from encoded plaintexts {(g, b): tensor}"""

    def __init__(self, ctx, level, gs, bs, pts, stream=None):
        self.ctx = ctx
        h = ctypes.c_void_p()
        parr = (ctypes.c_void_p * (len(gs) * len(bs)))(*[
            pts[(g, b)].data_ptr() if (g, b) in pts else None
            for g in gs for b in bs])
        _check(lib.chd_hoist_create(
            ctypes.byref(h), ctx.h, level, len(gs),
            (ctypes.c_int * len(gs))(*gs), len(bs),
            (ctypes.c_int * len(bs))(*bs), parr,
            stream if stream is not None else current_stream()))
        _own(self, h, lib.chd_hoist_destroy)

    @classmethod
    def from_messages(cls, ctx, level, pt_scale, gs, bs, msgs,
                      suppress_bs_swap=False, stream=None):
        """the reference's message constructor: msgs {(g, b): complex
        array}, encoded by the library"""
        self = cls.__new__(cls)
        self.ctx = ctx
        keys = [(g, b) for g in gs for b in bs]
        parts = {k: _split(msgs[k]) for k in keys if k in msgs}
        self._keep = parts
        re = (ctypes.c_void_p * len(keys))(*[
            parts[k][0].ctypes.data if k in parts else None for k in keys])
        im = (ctypes.c_void_p * len(keys))(*[
            parts[k][1].ctypes.data if k in parts else None for k in keys])
        ln = (ctypes.c_int * len(keys))(*[
            parts[k][0].size if k in parts else 0 for k in keys])
        h = ctypes.c_void_p()
        _check(lib.chd_hoist_create_from_messages(
            ctypes.byref(h), ctx.h, level, pt_scale, len(gs),
            (ctypes.c_int * len(gs))(*gs), len(bs),
            (ctypes.c_int * len(bs))(*bs), re, im, ln,
            1 if suppress_bs_swap else 0,
            stream if stream is not None else current_stream()))
        _own(self, h, lib.chd_hoist_destroy)
        return self


    @classmethod
    def linear_transform(cls, ctx, level, pt_scale, dim, diags, bs, gs=1,
                         pre_rotation=0, additional_pt_rot=0, stream=None):
        """LinearTransform of a dim x dim matrix given by its generalised
        diagonals {i: complex array of dim values}"""
        self = cls.__new__(cls)
        self.ctx = ctx
        idx = sorted(diags)
        parts = [_split(diags[i]) for i in idx]
        self._keep = parts
        re = (ctypes.c_void_p * len(idx))(*[p[0].ctypes.data for p in parts])
        im = (ctypes.c_void_p * len(idx))(*[p[1].ctypes.data for p in parts])
        h = ctypes.c_void_p()
        _check(lib.chd_linear_transform_create(
            ctypes.byref(h), ctx.h, level, pt_scale, dim, len(idx),
            (ctypes.c_int * len(idx))(*idx), re, im, bs, gs, pre_rotation,
            additional_pt_rot,
            stream if stream is not None else current_stream()))
        _own(self, h, lib.chd_hoist_destroy)
        return self

    def required_rotations(self, min_ks=False):
        n = lib.chd_hoist_required_rotations(self.h, int(min_ks), None, 0)
        if n < 0:
            _check(n)
        out = (ctypes.c_int * max(n, 1))()
        lib.chd_hoist_required_rotations(self.h, int(min_ks), out, n)
        return list(out[:n])

    def run(self, res, ct, keys, min_ks=False, stream=None):
        kr, kb, ka, nk, beta = Context._keys(keys)
        fn = lib.chd_hoist_run_min_ks if min_ks else lib.chd_hoist_run
        _check(fn(
            self.h, ptr(res[0]), ptr(res[1]), ptr(ct[0]), ptr(ct[1]), nk, kr,
            kb, ka, beta, stream if stream is not None else current_stream()))
