"""Python binding of the MI355X hybrid-attention engine (libha.so, C ABI in include/ha.h).

This mirrors the reference engine's host API for the token-mixer path (web/public/engine/engine.js):
``Engine(...)`` plays ``Engine.create`` / the constructor (engine.js:63-111), ``Engine.forward`` takes the
reference's option names ``cache`` / ``keep_cache`` / ``timestamps`` (engine.js:313) and returns a dict with
``cache`` (a :class:`Snapshot`, engine.js:349-362) and ``gpu_ms``; ``Snapshot.release()`` is engine.js:361.
Errors raise :class:`HAError`, as the reference throws ``Error``.

Tensors handed to :meth:`Engine.forward` are device buffers: any object with ``data_ptr()`` (a torch tensor on
the GPU) or a raw device address as ``int``. There is no CPU path: loading fails loudly if libha.so is missing.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libha.so")

HA_OK, HA_ERR_ARG, HA_ERR_CONTEXT, HA_ERR_HANDLE, HA_ERR_DEVICE, HA_ERR_NOMEM, HA_ERR_PARAM = 0, -1, -2, -3, -4, -5, -6
LINEAR, FULL, ADAPTER = 0, 1, 2  # ADAPTER: no token mixer (engine.js:256-261); its forward buffers may be None
F32, F16 = 0, 1
CHUNKED, SEQUENTIAL, CHUNKED_FUSED, CHUNKED_SPLIT, CHUNKED_PAIRED = 0, 1, 2, 3, 4
KIND_NAMES = {"linear_attention": LINEAR, "full_attention": FULL, "adapter": ADAPTER}


class HAError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("%s (ha status %d)" % (msg, code))
        self.code = code


class HaConfig(ctypes.Structure):
    _fields_ = [("n_layers", ctypes.c_int), ("layer_kind", ctypes.POINTER(ctypes.c_ubyte)),
                ("batch", ctypes.c_int), ("max_ctx", ctypes.c_int),
                ("H", ctypes.c_int), ("DK", ctypes.c_int), ("DV", ctypes.c_int), ("conv_k", ctypes.c_int),
                ("lin_stride", ctypes.c_int), ("lin_dtype", ctypes.c_int), ("lin_gnorm", ctypes.c_int),
                ("HQ", ctypes.c_int), ("HK", ctypes.c_int), ("HD", ctypes.c_int), ("rot_dim", ctypes.c_int),
                ("full_stride", ctypes.c_int), ("full_dtype", ctypes.c_int),
                ("rope_theta", ctypes.c_float), ("eps", ctypes.c_float)]


class HaMnbFormat(ctypes.Structure):
    _fields_ = [("bits", ctypes.c_int), ("group", ctypes.c_int), ("asym", ctypes.c_int)]


class HaForwardOpts(ctypes.Structure):
    _fields_ = [("recurrence", ctypes.c_int), ("timestamps", ctypes.c_int), ("sync", ctypes.c_int),
                ("gpu_ms", ctypes.c_float), ("layer_ms", ctypes.POINTER(ctypes.c_float)),
                ("mixer_ms", ctypes.POINTER(ctypes.c_float)), ("debug_unpublished_waits", ctypes.c_int)]


_lib = None


def load_library(path=LIB_PATH):
    """Load libha.so once; raise if it has not been built (there is no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError("libha.so is not built at %s; run __graft_entry__.build()" % path)
    lib = ctypes.CDLL(path)
    vp, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    sig = {
        "ha_last_error": ([], ctypes.c_char_p),
        "ha_abi_version": ([], i),
        "ha_create": ([ctypes.POINTER(HaConfig), i, ctypes.POINTER(vp)], i),
        "ha_destroy": ([vp], i),
        "ha_set_stream": ([vp, vp], i),
        "ha_share_scratch": ([vp, vp], i),
        "ha_set_param": ([vp, i, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float), sz], i),
        "ha_forward": ([vp, i, ctypes.POINTER(vp), ctypes.POINTER(vp), vp, ctypes.POINTER(vp),
                        ctypes.POINTER(HaForwardOpts)], i),
        "ha_snapshot_tokens": ([vp, ctypes.POINTER(i)], i),
        "ha_snapshot_layout": ([vp, ctypes.POINTER(i), ctypes.POINTER(i)], i),
        "ha_snapshot_read": ([vp, i, ctypes.c_char_p, vp, sz], i),
        "ha_snapshot_release": ([vp], i),
        "ha_snapshot_destroy": ([vp], i),
        "ha_device_alloc": ([vp, sz, ctypes.POINTER(vp)], i),
        "ha_device_free": ([vp, vp], i),
        "ha_copy_to_device": ([vp, vp, vp, sz], i),
        "ha_copy_to_host": ([vp, vp, vp, sz], i),
        "ha_synchronize": ([vp], i),
        "ha_mnb_create": ([i, i, ctypes.POINTER(HaMnbFormat), vp, vp, vp, i, ctypes.POINTER(vp)], i),
        "ha_mnb_forward": ([vp, i, vp, vp, vp], i),
        "ha_mnb_forward_noalloc": ([vp, i, vp, vp, vp], i),
        "ha_mnb_destroy": ([vp], i),
        "ha_fwht": ([vp, ctypes.c_long, i, i, vp], i),
        "ha_embed": ([vp, i, vp, vp, vp], i),
        "ha_add_norm": ([i, i, i, vp, vp, vp, vp, i, vp, ctypes.c_float, i, vp], i),
        "ha_silu_mul": ([i, i, vp, vp, i, vp], i),
        "ha_add_bias": ([i, i, vp, vp, i, vp], i),
        "ha_timer_create": ([i, i, ctypes.POINTER(vp)], i),
        "ha_timer_mark": ([vp, i, vp], i),
        "ha_timer_elapsed": ([vp, i, i, ctypes.POINTER(ctypes.c_float)], i),
        "ha_timer_destroy": ([vp], i),
    }
    for name, (args, res) in sig.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = res
    _lib = lib
    return lib


def _check(rc):
    if rc != HA_OK:
        raise HAError(rc, _lib.ha_last_error().decode())


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def model_config(layer_types, batch=1, max_ctx=4096, lin_dtype=F32, full_dtype=F16, lin_gnorm=True, **kw):
    """Engine shape for the Qwen3.5-2B torso (the reference's manifest config, export_engine.py:83)."""
    d = dict(H=16, DK=128, DV=128, conv_k=4, lin_stride=8256, HQ=8, HK=2, HD=256, rot_dim=64,
             full_stride=5120, rope_theta=1e7, eps=1e-6)
    d.update(kw)
    kinds = [KIND_NAMES[k] if isinstance(k, str) else int(k) for k in layer_types]
    return dict(kinds=kinds, batch=batch, max_ctx=max_ctx, lin_dtype=lin_dtype, full_dtype=full_dtype,
                lin_gnorm=int(bool(lin_gnorm)), **d)


class Snapshot:
    """A prefix-cache snapshot (engine.js:352): ``P`` tokens of state, raw tail rows and K/V."""

    def __init__(self, engine, handle):
        self.engine = engine
        self._h = ctypes.c_void_p(handle)
        p = ctypes.c_int()
        _check(_lib.ha_snapshot_tokens(self._h, ctypes.byref(p)))
        self.P = p.value
        sp, tr = ctypes.c_int(), ctypes.c_int()
        _check(_lib.ha_snapshot_layout(self._h, ctypes.byref(sp), ctypes.byref(tr)))
        self.state_pos, self.tail_rows = sp.value, tr.value

    @property
    def handle(self):
        return self._h

    def read(self, layer, what, out):
        """Copy a part ("state", "tail", "K", "V") into the numpy array ``out`` (exact byte size)."""
        _check(_lib.ha_snapshot_read(self._h, layer, what.encode(), out.ctypes.data, out.nbytes))
        return out

    def release(self):
        _check(_lib.ha_snapshot_release(self._h))

    def __del__(self):
        try:
            if self._h and _lib is not None:
                _lib.ha_snapshot_destroy(self._h)
                self._h = None
        except Exception:
            pass


class Engine:
    """Hybrid-attention engine bound to one HIP device and stream (engine.js:61-111 facade)."""

    def __init__(self, cfg, device=0, stream=None):
        lib = load_library()
        self.cfg = dict(cfg)
        kinds = (ctypes.c_ubyte * len(cfg["kinds"]))(*cfg["kinds"])
        self._kinds = kinds
        c = HaConfig(n_layers=len(cfg["kinds"]), layer_kind=kinds, batch=cfg["batch"], max_ctx=cfg["max_ctx"],
                     H=cfg["H"], DK=cfg["DK"], DV=cfg["DV"], conv_k=cfg["conv_k"], lin_stride=cfg["lin_stride"],
                     lin_dtype=cfg["lin_dtype"], lin_gnorm=cfg["lin_gnorm"], HQ=cfg["HQ"], HK=cfg["HK"],
                     HD=cfg["HD"], rot_dim=cfg["rot_dim"], full_stride=cfg["full_stride"],
                     full_dtype=cfg["full_dtype"], rope_theta=cfg["rope_theta"], eps=cfg["eps"])
        h = ctypes.c_void_p()
        _check(lib.ha_create(ctypes.byref(c), device, ctypes.byref(h)))
        self._h = h
        self.n_layers = len(cfg["kinds"])
        if stream is not None:
            self.set_stream(stream)

    def set_stream(self, stream):
        _check(_lib.ha_set_stream(self._h, ctypes.c_void_p(stream) if stream else None))

    def share_scratch(self, holder):
        """Use `holder`'s call-time device buffers (ha_share_scratch); both engines must already run on one stream
        (set_stream), so that their calls never overlap."""
        _check(_lib.ha_share_scratch(self._h, holder._h))

    def set_param(self, layer, name, values):
        import numpy as np
        a = np.ascontiguousarray(values, dtype=np.float32).ravel()
        _check(_lib.ha_set_param(self._h, layer, name.encode(), a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                 a.size))

    def forward(self, L, layer_in, layer_out, cache=None, keep_cache=False, recurrence=CHUNKED, timestamps=False,
                layer_ms=False, sync=False, mixer_ms=False, debug_unpublished_waits=False):
        """ha_forward. layer_ms / mixer_ms add per-layer GPU times (with / without the raw-row tail copy) to the
        result; debug_unpublished_waits is the test-only option of ha_forward_opts (the call then fails with
        HA_ERR_DEVICE once it is waited for)."""
        n = self.n_layers
        ins = (ctypes.c_void_p * n)(*[_ptr(x) for x in layer_in])
        outs = (ctypes.c_void_p * n)(*[_ptr(x) for x in layer_out])
        lm = (ctypes.c_float * n)() if layer_ms else None
        mm = (ctypes.c_float * n)() if mixer_ms else None
        opts = HaForwardOpts(recurrence=recurrence, timestamps=int(timestamps), sync=int(sync), gpu_ms=0.0,
                             layer_ms=lm, mixer_ms=mm, debug_unpublished_waits=int(bool(debug_unpublished_waits)))
        keep = ctypes.c_void_p() if keep_cache else None
        rc = _lib.ha_forward(self._h, L, ins, outs, cache.handle if cache is not None else None,
                             ctypes.byref(keep) if keep_cache else None, ctypes.byref(opts))
        _check(rc)
        res = {"cache": Snapshot(self, keep.value) if keep_cache else None}
        if timestamps:
            res["gpu_ms"] = opts.gpu_ms
        if layer_ms:
            res["layer_ms"] = list(lm)
        if mixer_ms:
            res["mixer_ms"] = list(mm)
        return res

    def synchronize(self):
        _check(_lib.ha_synchronize(self._h))

    def close(self):
        if self._h:
            _check(_lib.ha_destroy(self._h))
            self._h = None

    def __del__(self):
        try:
            if self._h and _lib is not None:
                _lib.ha_destroy(self._h)
                self._h = None
        except Exception:
            pass


class MnbWeight:
    """A MatMulNBits weight matrix on the GPU (formats of web/public/gemmbench/kernels.js:1-14): ``q`` packed blocks
    [N][K/32][bits] u32, ``s`` f16 scales [N][K/group], ``b`` f16 biases (asymmetric). The device buffers are the
    caller's (the handle borrows them); this wrapper keeps a reference to q, s and b for its own lifetime.
    ``forward(M, a, y)`` computes y[M][N] = a[M][K] x W^T in f16 (engine.js:236-246)."""

    def __init__(self, N, K, q, s, b=None, bits=4, group=32, asym=False, device=0):
        load_library()
        self.N, self.K, self.bits, self.group, self.asym = N, K, bits, group, bool(asym)
        fmt = HaMnbFormat(bits, group, int(bool(asym)))
        h = ctypes.c_void_p()
        _check(_lib.ha_mnb_create(N, K, ctypes.byref(fmt), _ptr(q), _ptr(s), _ptr(b), device, ctypes.byref(h)))
        self._h = h
        self._borrowed = (q, s, b)

    def forward(self, M, a, y, stream=None):
        _check(_lib.ha_mnb_forward(self._h, M, _ptr(a), _ptr(y), _ptr(stream) if stream is not None else None))

    def forward_noalloc(self, M, a, y, stream=None):
        """forward() without any device allocation: split-K partials go to the library's fixed per-GPU scratch
        (ha_mnb_forward_noalloc; calls that overlap on one GPU race)."""
        _check(_lib.ha_mnb_forward_noalloc(self._h, M, _ptr(a), _ptr(y), _ptr(stream) if stream is not None else None))

    def close(self):
        if self._h:
            _check(_lib.ha_mnb_destroy(self._h))
            self._h = None
            self._borrowed = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def fwht(x, elems, n, device=0, stream=None):
    """In-place orthonormal Walsh-Hadamard transform of each n-block of the f16 device array x (wgsl.js:94-110)."""
    load_library()
    _check(_lib.ha_fwht(_ptr(x), elems, n, device, _ptr(stream) if stream is not None else None))


def _st(stream):
    return _ptr(stream) if stream is not None else None


def embed(table, L, ids, x, stream=None):
    """x[t] = f32 row ids[t] of the quantised embedding table `table` (an MnbWeight with N = table rows, K = hidden
    size; wgsl.js:33-52). ids: L u32 on the device; an id outside the table gives a NaN row."""
    load_library()
    _check(_lib.ha_embed(table._h, L, _ptr(ids), _ptr(x), _st(stream)))


def add_norm(R, D, nx, x, y, w, h, out_f32=False, rows=None, eps=1e-6, device=0, stream=None):
    """Residual add (x[s] += y[s] when y is given) then RMSNorm h[r] = x[s] rsqrt(mean(x[s]^2) + eps) w, with
    s = rows[r] (identity when rows is None); h f16, or f32 with out_f32 (wgsl.js:55-78)."""
    load_library()
    _check(_lib.ha_add_norm(R, D, nx, _ptr(x), _ptr(y), _ptr(w), _ptr(h), int(bool(out_f32)), _ptr(rows), eps,
                            device, _st(stream)))


def silu_mul(L, I, big, mid, device=0, stream=None):
    """mid[t][j] = silu(big[t][j]) * big[t][I + j] (f16; wgsl.js:81-90)."""
    load_library()
    _check(_lib.ha_silu_mul(L, I, _ptr(big), _ptr(mid), device, _st(stream)))


def add_bias(L, N, y, c, device=0, stream=None):
    """y[t][j] += c[j] (y f16, c f32; wgsl.js:113-121)."""
    load_library()
    _check(_lib.ha_add_bias(L, N, _ptr(y), _ptr(c), device, _st(stream)))


class Timer:
    """n GPU timestamps (ha_timer_*): the counterpart of a WebGPU timestamp query set."""

    def __init__(self, n, device=0):
        lib = load_library()
        h = ctypes.c_void_p()
        _check(lib.ha_timer_create(device, n, ctypes.byref(h)))
        self._h = h

    def mark(self, i, stream=None):
        _check(_lib.ha_timer_mark(self._h, i, _st(stream)))

    def elapsed(self, i, j):
        ms = ctypes.c_float()
        _check(_lib.ha_timer_elapsed(self._h, i, j, ctypes.byref(ms)))
        return ms.value

    def close(self):
        if self._h:
            _check(_lib.ha_timer_destroy(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Torso:
    """The whole torso forward (web/public/engine/engine.js:247-285, 313-376), batch 1, from the C ABI calls js/engine.js
    Torso makes, in the same order, on one stream: EMBED; per layer the input norm (residual add from layer 1 on),
    in_proj / qkv, the layer's token mixer (an Engine of its own), out_proj / o_proj, the post norm, gate_up,
    SILU_MUL, down (an adapter layer: proj + bias); the final norm of the requested rows in f32.

    set_weight(name, MnbWeight) for the quantised tensors ("embed", "layers.<i>.in_proj" | "qkv" | "out_proj" |
    "o_proj" | "gate_up" | "down" | "proj"); set_param(name, f32 array) for "final_norm", "layers.<i>.in_norm" |
    "post_norm" | "bias" and the mixers' "conv" | "neg_exp_A" | "dt_bias" | "gnorm" | "q_norm" | "k_norm"."""

    _MIXER = ("conv", "neg_exp_A", "dt_bias", "gnorm", "q_norm", "k_norm")

    def __init__(self, layer_types, D=2048, I=6144, max_ctx=4096, device=0):
        import torch
        self.torch = torch
        self.types, self.D, self.I, self.device = list(layer_types), D, I, device
        self.dev = "cuda:%d" % device
        self.stream = torch.cuda.Stream(device=self.dev)
        self.st = self.stream.cuda_stream
        self.mix = {i: Engine(model_config([t], batch=1, max_ctx=max_ctx, lin_dtype=F16, full_dtype=F16),
                              device=device, stream=self.st)
                    for i, t in enumerate(self.types) if t != "adapter"}
        engines = list(self.mix.values())
        for m in engines[1:]:  # one stream orders every call, so one set of call-time buffers serves all
            m.share_scratch(engines[0])
        self.w, self.v = {}, {}
        self._prof, self.diag = None, {}

    def set_weight(self, name, w):
        self.w[name] = w

    def set_param(self, name, data):
        parts = name.split(".")
        if len(parts) == 3 and parts[0] == "layers" and parts[2] in self._MIXER:
            self.mix[int(parts[1])].set_param(0, parts[2], data)
            return
        self.v[name] = self.torch.as_tensor(data, dtype=self.torch.float32).to(self.dev)

    def _step(self, label, fn):
        pr = self._prof
        if pr is None:
            return fn()
        k = len(pr["labels"])
        pr["timer"].mark(2 * k, self.st)
        r = fn()
        pr["timer"].mark(2 * k + 1, self.st)
        pr["labels"].append(label)
        return r

    def forward(self, ids, rows=None, cache=None, keep=False, timestamps=False, debug_layers=False):
        """ids: token rows of the embedding table; rows: indices into ids to return (default all). Returns
        (hidden f32 [len(rows)][D] on the host, {layer: Snapshot} when keep). The reference's diagnostics
        (engine.js:313-376) go to self.diag: "gpu_ms" (timestamps: GPU time from the embedding to the final norm) and
        "layers" (debug_layers: the residual stream x entering each layer i >= 1, f32 [L][D], read back between the
        layers)."""
        import numpy as np
        torch, D, I, st = self.torch, self.D, self.I, self.st
        L = len(ids)
        rows = list(range(L)) if rows is None else list(rows)
        f16, f32 = torch.float16, torch.float32
        maxN = max([2 * I] + [w.N for w in self.w.values()])
        step = self._step
        self.diag = {}
        timer = Timer(2, self.device) if timestamps else None
        layers = []
        with torch.cuda.stream(self.stream):
            idd = torch.as_tensor(np.asarray(ids, np.uint32).view(np.int32)).to(self.dev)
            x = torch.empty(L, D, dtype=f32, device=self.dev)
            h = torch.empty(L, D, dtype=f16, device=self.dev)
            big = torch.empty(L, maxN, dtype=f16, device=self.dev)
            o = torch.empty(L, D, dtype=f16, device=self.dev)
            y = torch.empty(L, D, dtype=f16, device=self.dev)
            mid = torch.empty(L, I, dtype=f16, device=self.dev)
            rd = torch.as_tensor(np.asarray(rows or [0], np.uint32).view(np.int32)).to(self.dev)
            out = torch.empty(len(rows), D, dtype=f32, device=self.dev)
            if timer:
                timer.mark(0, st)
            step("embed", lambda: embed(self.w["embed"], L, idd, x, stream=st))
            snaps = {}
            for i, t in enumerate(self.types):
                p, S = "layers.%d." % i, "L%d/" % i
                step(S + "in_norm", lambda: add_norm(L, D, L, x, y if i > 0 else None, self.v[p + "in_norm"], h,
                                                     device=self.device, stream=st))
                if debug_layers and i > 0:
                    self.stream.synchronize()
                    layers.append(x.cpu().numpy())
                if t == "adapter":
                    step(S + "proj", lambda: self.w[p + "proj"].forward(L, h, y, st))
                    step(S + "bias", lambda: add_bias(L, D, y, self.v[p + "bias"], device=self.device, stream=st))
                    continue
                lin = t == "linear_attention"
                step(S + ("in_proj" if lin else "qkv"),
                     lambda: self.w[p + ("in_proj" if lin else "qkv")].forward(L, h, big, st))
                r = step(S + ("gdn" if lin else "attn"),
                         lambda: self.mix[i].forward(L, [big], [o], cache=cache[i] if cache else None, keep_cache=keep))
                snaps[i] = r["cache"]
                step(S + ("out_proj" if lin else "o_proj"),
                     lambda: self.w[p + ("out_proj" if lin else "o_proj")].forward(L, o, y, st))
                step(S + "post_norm", lambda: add_norm(L, D, L, x, y, self.v[p + "post_norm"], h, device=self.device,
                                                       stream=st))
                step(S + "gate_up", lambda: self.w[p + "gate_up"].forward(L, h, big, st))
                step(S + "silu", lambda: silu_mul(L, I, big, mid, device=self.device, stream=st))
                step(S + "down", lambda: self.w[p + "down"].forward(L, mid, y, st))
            if rows:
                step("final_norm", lambda: add_norm(len(rows), D, L, x, y, self.v["final_norm"], out, out_f32=True,
                                                    rows=rd, device=self.device, stream=st))
            if timer:
                timer.mark(1, st)
        self.stream.synchronize()
        if timer:
            self.diag["gpu_ms"] = timer.elapsed(0, 1)
            timer.close()
        if debug_layers:
            self.diag["layers"] = layers
        return out.cpu().numpy(), (snaps if keep else None)

    def profile(self, ids, cache=None):
        """GPU time of every step of a forward over ids, summed over the layers by the step's name without its layer
        prefix, in ms to 2 decimals, largest first (engine.js:292-307). A timestamp pair brackets every step."""
        cap = 2 * (3 + 16 * len(self.types))
        self._prof = {"timer": Timer(cap, self.device), "labels": []}
        try:
            self.forward(ids, [], cache=cache)
            by = {}
            for k, label in enumerate(self._prof["labels"]):
                name = label.split("/", 1)[1] if label.startswith("L") and "/" in label else label
                by[name] = by.get(name, 0.0) + self._prof["timer"].elapsed(2 * k, 2 * k + 1)
            return {k: round(v, 2) for k, v in sorted(by.items(), key=lambda kv: -kv[1])}
        finally:
            self._prof["timer"].close()
            self._prof = None
