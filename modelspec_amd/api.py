"""ctypes bindings of libmsx.so (include/msx.h).

Loading fails loudly when the library is missing: there is no CPU fallback in this package.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmsx.so")

CONFIGS = ("linear_regression", "mnist_mlp", "mlp_classifier", "transformer_block", "bert_tiny",
           "bert_cpu", "bert_micro", "block_micro", "mlp_micro", "bert_base", "bert_micro_mixed", "bert_mini_mixed")

STATUS = {0: "ok", -1: "invalid", -2: "data", -3: "device", -4: "nonfinite", -5: "unsupported", -6: "checkpoint",
          -7: "artifact"}


class MsxError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"{STATUS.get(code, code)}: {message}")
        self.code = code


class Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int32), ("data", ctypes.c_void_p),
                ("count", ctypes.c_uint64)]


class RunStats(ctypes.Structure):
    _fields_ = [("steps", ctypes.c_uint64), ("graph_launches", ctypes.c_uint64),
                ("kernels_per_step", ctypes.c_uint64), ("bytes_uploaded", ctypes.c_uint64),
                ("device_bytes", ctypes.c_uint64)]


class HeldOutMetrics(ctypes.Structure):
    _fields_ = [("loss", ctypes.c_float), ("accuracy", ctypes.c_float), ("numerator", ctypes.c_double),
                ("denominator", ctypes.c_double), ("correct", ctypes.c_uint64), ("selected", ctypes.c_uint64)]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MsxError(-3, f"{LIB_PATH} is not built: run `python -m modelspec_amd.build` (hipcc, gfx950)")
        L = ctypes.CDLL(LIB_PATH)
        vp, c64, u64, u32, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int32
        L.msx_last_error.restype = ctypes.c_char_p
        L.msx_compile_config.argtypes = [ctypes.c_char_p, c64, c64, ctypes.POINTER(vp), ctypes.POINTER(vp)]
        L.msx_free.argtypes = [vp]
        L.msx_open.argtypes = [ctypes.c_int, ctypes.POINTER(vp)]
        L.msx_close.argtypes = [vp]
        L.msx_load.argtypes = [vp, ctypes.c_char_p, ctypes.c_char_p, u64, u32]
        L.msx_set_params.argtypes = [vp, ctypes.POINTER(vp), ctypes.POINTER(u64), u32]
        L.msx_read_param.argtypes = [vp, u32, vp, u64]
        L.msx_read_moment.argtypes = [vp, u32, i32, vp, u64]
        L.msx_run_steps.argtypes = [vp, u32, ctypes.POINTER(ctypes.POINTER(Tensor)), ctypes.POINTER(u32), vp]
        L.msx_forward.argtypes = [vp, ctypes.POINTER(Tensor), u32, vp, vp, u64]
        L.msx_stats.argtypes = [vp, ctypes.POINTER(RunStats)]
        L.msx_train_config.argtypes = [vp, ctypes.c_char_p, c64, c64, vp, u64, vp, u64, ctypes.POINTER(ctypes.c_double)]
        L.msx_evaluate.argtypes = [vp, u32, ctypes.POINTER(ctypes.POINTER(Tensor)), ctypes.POINTER(u32),
                                   ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(HeldOutMetrics)]
        L.msx_evaluate_static.argtypes = L.msx_evaluate.argtypes
        L.msx_set_fusion.argtypes = [vp, u32]
        L.msx_plan.argtypes = [ctypes.c_char_p, ctypes.c_char_p, u32, ctypes.c_int32, ctypes.POINTER(ctypes.c_void_p)]
        L.msx_train_config_eval.argtypes = [vp, ctypes.c_char_p, c64, u64, u64, vp, u64, vp,
                                            ctypes.POINTER(HeldOutMetrics), u64, ctypes.POINTER(u64),
                                            ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]
        L.msx_load_packed.argtypes = [vp, ctypes.c_char_p]
        L.msx_write_packed.argtypes = [ctypes.c_char_p, vp, u64, vp, u64, u64, u64, ctypes.c_char_p, ctypes.c_char_p,
                                       ctypes.c_double]
        L.msx_train_packed.argtypes = [vp, ctypes.c_char_p, ctypes.c_char_p, c64, u64, u64, vp, u64, vp, u64, vp,
                                       ctypes.POINTER(HeldOutMetrics), u64, ctypes.POINTER(u64),
                                       ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]
        L.msx_read_input.argtypes = [vp, i32, ctypes.c_char_p, vp, u64]
        L.msx_set_precision.argtypes = [vp, i32, ctypes.c_float, u32]
        L.msx_loss_scale.argtypes = [vp, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(u64)]
        L.msx_checkpoint_write.argtypes = [vp, ctypes.c_char_p, u64]
        L.msx_write_artifact.argtypes = [vp, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p]
        L.msx_load_artifact.argtypes = [vp, ctypes.c_char_p, u64]
        L.msx_check_artifact.argtypes = [ctypes.c_char_p, ctypes.c_char_p]
        L.msx_checkpoint_read.argtypes = [vp, ctypes.c_char_p, i32, ctypes.POINTER(u64)]
        L.msx_train_checkpointed.argtypes = [vp, ctypes.c_char_p, ctypes.c_char_p, c64, ctypes.c_char_p, u64,
                                             ctypes.c_char_p, vp, u64, vp, u64, ctypes.POINTER(u64)]
        L.msx_prog_new.argtypes = [vp, ctypes.c_char_p, u64, ctypes.POINTER(vp)]
        L.msx_prog_run.argtypes = [vp, ctypes.POINTER(Tensor), u32, ctypes.POINTER(vp), ctypes.POINTER(u64), u32]
        L.msx_prog_output.argtypes = [vp, u32, vp, u64]
        L.msx_prog_free.argtypes = [vp]
        _lib = L
    return _lib


def _check(rc):
    if rc != 0:
        raise MsxError(rc, lib().msx_last_error().decode())


def device_count():
    return lib().msx_device_count()


CONFIG_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "configs")


def config_file(name):
    """The path of the .mspec source of a config this package ships (modelspec_amd/configs)."""
    return os.path.join(CONFIG_DIR, name + ".mspec")


def plan(step_ir, forward_ir, prediction_output=1, mixed=False):
    """This backend's launch and buffer plans of a step and its forward program (msx_plan; no
    device needed)."""
    out = ctypes.c_void_p()
    _check(lib().msx_plan(step_ir.encode(), forward_ir.encode(), prediction_output, 1 if mixed else 0,
                          ctypes.byref(out)))
    try:
        return ctypes.string_at(out).decode()
    finally:
        lib().msx_free(out)


def compile_config(name, masked_rows=-1, steps=-1):
    """The printed training step and forward program of a built-in config, or of the .mspec source
    at the path `name` (a name ending in ".mspec")."""
    s, f = ctypes.c_void_p(), ctypes.c_void_p()
    _check(lib().msx_compile_config(name.encode(), masked_rows, steps, ctypes.byref(s), ctypes.byref(f)))
    try:
        return ctypes.string_at(s).decode(), ctypes.string_at(f).decode()
    finally:
        lib().msx_free(s)
        lib().msx_free(f)


def _tensors(named):
    """(ctypes array, keepalive) of msx_tensor from {name: ndarray}."""
    keep, arr = [], (Tensor * max(1, len(named)))()
    for i, (name, a) in enumerate(named.items()):
        a = np.ascontiguousarray(a)
        if a.dtype == np.float32:
            dt = 0
        elif a.dtype == np.int32:
            dt = 1
        else:
            raise TypeError(f"input {name}: dtype {a.dtype} is neither float32 nor int32")
        nb = name.encode()
        keep += [a, nb]
        arr[i] = Tensor(nb, dt, a.ctypes.data, a.size)
    return arr, keep


class Program:
    """One Tensor IR program on the device (per-op parity tests)."""

    def __init__(self, ctx, text, seed=0):
        self._h = ctypes.c_void_p()
        _check(lib().msx_prog_new(ctx._h, text.encode(), seed, ctypes.byref(self._h)))

    def run(self, inputs, params=()):
        arr, keep = _tensors(inputs)
        ps = [np.ascontiguousarray(p, np.float32) for p in params]
        pv = (ctypes.c_void_p * max(1, len(ps)))(*[p.ctypes.data for p in ps])
        pc = (ctypes.c_uint64 * max(1, len(ps)))(*[p.size for p in ps])
        _check(lib().msx_prog_run(self._h, arr, len(inputs), pv, pc, len(ps)))

    def output(self, k, count):
        out = np.empty(count, np.float32)
        _check(lib().msx_prog_output(self._h, k, out.ctypes.data, count))
        return out

    def close(self):
        if self._h:
            lib().msx_prog_free(self._h)
            self._h = None

    def __del__(self):
        self.close()


class Context:
    """A device context: msx_open / msx_close."""

    def __init__(self, device=0):
        self._h = ctypes.c_void_p()
        _check(lib().msx_open(device, ctypes.byref(self._h)))

    def close(self):
        if self._h:
            lib().msx_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def load(self, step_ir, forward_ir, seed, prediction_output=1):
        _check(lib().msx_load(self._h, step_ir.encode(), forward_ir.encode(), seed, prediction_output))

    def set_params(self, values):
        vs = [np.ascontiguousarray(v, np.float32) for v in values]
        pv = (ctypes.c_void_p * len(vs))(*[v.ctypes.data for v in vs])
        pc = (ctypes.c_uint64 * len(vs))(*[v.size for v in vs])
        _check(lib().msx_set_params(self._h, pv, pc, len(vs)))

    def read_param(self, k, count):
        out = np.empty(count, np.float32)
        _check(lib().msx_read_param(self._h, k, out.ctypes.data, count))
        return out

    def read_moment(self, k, which, count):
        out = np.empty(count, np.float32)
        _check(lib().msx_read_moment(self._h, k, ord(which), out.ctypes.data, count))
        return out

    @staticmethod
    def _batches(per_step):
        n = len(per_step)
        arrs, keep = [], []
        for named in per_step:
            a, k = _tensors(named)
            arrs.append(a)
            keep += k
        ptrs = (ctypes.POINTER(Tensor) * max(1, n))(*[ctypes.cast(a, ctypes.POINTER(Tensor)) for a in arrs])
        counts = (ctypes.c_uint32 * max(1, n))(*[len(d) for d in per_step])
        return ptrs, counts, (arrs, keep)

    def run_steps(self, per_step):
        """per_step: list of {name: ndarray}; returns the losses."""
        n = len(per_step)
        ptrs, counts, keep = self._batches(per_step)
        losses = np.empty(n, np.float32)
        _check(lib().msx_run_steps(self._h, n, ptrs, counts, losses.ctypes.data))
        return losses

    def forward(self, inputs, prediction_count=0):
        arr, keep = _tensors(inputs)
        loss = ctypes.c_float()
        pred = np.empty(prediction_count, np.float32) if prediction_count else None
        _check(lib().msx_forward(self._h, arr, len(inputs), ctypes.addressof(loss),
                                 pred.ctypes.data if pred is not None else None, prediction_count))
        return loss.value, pred

    def evaluate(self, batches, labels, weights):
        """Held-out metrics of the forward program on the current parameters over `batches`
        ({name: ndarray} each): a dict of loss, accuracy, numerator, denominator, correct, selected."""
        ptrs, counts, keep = self._batches(batches)
        out = HeldOutMetrics()
        _check(lib().msx_evaluate(self._h, len(batches), ptrs, counts, labels.encode(), weights.encode(),
                                  ctypes.byref(out)))
        return out.as_dict()

    def evaluate_static(self, batches, labels, weights):
        """`evaluate` through msx_evaluate_static: no device allocation, at most 65,536 rows a batch."""
        ptrs, counts, keep = self._batches(batches)
        out = HeldOutMetrics()
        _check(lib().msx_evaluate_static(self._h, len(batches), ptrs, counts, labels.encode(), weights.encode(),
                                         ctypes.byref(out)))
        return out.as_dict()

    def train_config_eval(self, name, eval_every, eval_batches, steps=-1):
        """A synthetic run with held-out evaluation: (losses, [(step, metrics dict)], train s, eval s)."""
        n_steps = steps if steps >= 0 else config_steps(name)
        losses = np.zeros(n_steps + 1, np.float32)
        cap = n_steps // eval_every + 2
        at = np.zeros(cap, np.uint64)
        evals = (HeldOutMetrics * cap)()
        n, ts, es = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_double()
        _check(lib().msx_train_config_eval(self._h, name.encode(), steps, eval_every, eval_batches, losses.ctypes.data,
                                           losses.size, at.ctypes.data, evals, cap, ctypes.byref(n), ctypes.byref(ts),
                                           ctypes.byref(es)))
        return losses, [(int(at[k]), evals[k].as_dict()) for k in range(n.value)], ts.value, es.value

    def load_packed(self, path):
        """Binds a packed directory to the next load; None unbinds it."""
        _check(lib().msx_load_packed(self._h, None if path is None else str(path).encode()))

    def read_input(self, program, name, count, dtype=np.int32):
        """The device copy of an input of the step (program 0) or forward (1) program."""
        out = np.zeros(count, dtype)
        _check(lib().msx_read_input(self._h, program, name.encode(), out.ctypes.data, count))
        return out

    def train_packed(self, name, path, steps, eval_every=0, eval_batches=0):
        """A run of a built-in config on a packed directory: (losses, flat params, [(step, metrics)])."""
        step_ir, _ = compile_config(name, -1, steps)
        losses = np.zeros(steps + 1, np.float32)
        params = np.zeros(param_count(step_ir), np.float32)
        cap = (steps // eval_every + 2) if eval_every else 1
        at = np.zeros(cap, np.uint64)
        evals = (HeldOutMetrics * cap)()
        n, ts, es = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_double()
        _check(lib().msx_train_packed(self._h, name.encode(), str(path).encode(), steps, eval_every, eval_batches,
                                      losses.ctypes.data, losses.size, params.ctypes.data, params.size, at.ctypes.data,
                                      evals, cap, ctypes.byref(n), ctypes.byref(ts), ctypes.byref(es)))
        return losses, params, [(int(at[k]), evals[k].as_dict()) for k in range(n.value)]

    def write_artifact(self, path, source_text=None):
        """Writes the loaded step as a Hip artifact directory; returns the artifact hash."""
        out = ctypes.create_string_buffer(65)
        _check(lib().msx_write_artifact(self._h, str(path).encode(),
                                        None if source_text is None else source_text.encode(), out))
        return out.value.decode()

    def load_artifact(self, path, seed):
        _check(lib().msx_load_artifact(self._h, str(path).encode(), seed))

    def checkpoint_write(self, path, step):
        _check(lib().msx_checkpoint_write(self._h, str(path).encode(), step))

    def checkpoint_read(self, path, resume=True):
        """Uploads a checkpoint's parameters (and AdamW moments when resuming); returns its step."""
        step = ctypes.c_uint64()
        _check(lib().msx_checkpoint_read(self._h, str(path).encode(), int(resume), ctypes.byref(step)))
        return step.value

    def train_checkpointed(self, name, steps, packed=None, resume=None, every=0, path=None):
        """A run that may resume from a checkpoint and write checkpoints: (losses, params, start step)."""
        enc = lambda x: None if x is None else str(x).encode()
        step_ir, _ = compile_config(name)
        losses = np.zeros(steps + 1, np.float32)
        params = np.zeros(param_count(step_ir), np.float32)
        start = ctypes.c_uint64()
        _check(lib().msx_train_checkpointed(self._h, name.encode(), enc(packed), steps, enc(resume), every, enc(path),
                                            losses.ctypes.data, losses.size, params.ctypes.data, params.size,
                                            ctypes.byref(start)))
        return losses, params, start.value

    def set_fusion(self, ce_head=False, optimizer=True):
        """Optional fusions of the next load (msx_set_fusion): ce_head folds the cross-entropy into
        its decoder head GEMMs; optimizer (the default) runs the deferred column finalize inside
        the AdamW launch."""
        _check(lib().msx_set_fusion(self._h, (1 if ce_head else 0) | (2 if optimizer else 0)))

    def set_precision(self, mixed, loss_scale=65536.0, scale_window=2000):
        """The precision of the next load (and per-op program): f16 MFMA GEMMs with loss scaling."""
        _check(lib().msx_set_precision(self._h, int(mixed), loss_scale, scale_window))

    def loss_scale(self):
        """(current loss scale, steps skipped for an overflow) of the loaded step."""
        sc, sk = ctypes.c_float(), ctypes.c_uint64()
        _check(lib().msx_loss_scale(self._h, ctypes.byref(sc), ctypes.byref(sk)))
        return sc.value, sk.value

    def stats(self):
        s = RunStats()
        _check(lib().msx_stats(self._h, ctypes.byref(s)))
        return {f: getattr(s, f) for f, _ in RunStats._fields_}

    def train_config(self, name, steps=-1, masked_rows=-1, n_params=None):
        """A whole synthetic run of a built-in config: (losses[steps+1], flat params, seconds)."""
        step_ir, _ = compile_config(name, masked_rows, steps)
        if n_params is None:
            n_params = param_count(step_ir)
        n_steps = steps if steps >= 0 else config_steps(name)
        losses = np.zeros(n_steps + 1, np.float32)
        params = np.zeros(n_params, np.float32)
        secs = ctypes.c_double()
        _check(lib().msx_train_config(self._h, name.encode(), steps, masked_rows, losses.ctypes.data, losses.size,
                                      params.ctypes.data, params.size, ctypes.byref(secs)))
        return losses, params, secs.value

    def program(self, text, seed=0):
        return Program(self, text, seed)


DATASET_ID = "0c5a3f9e-2b71-8d40-9e6a-51f2c7d8a903"
TOKENIZER_ID = "7e19b4c2-a5d3-8f60-8b21-c4e7d9a0f518"


def write_packed(path, train, heldout, seq_len, vocabulary_size, dataset_id=DATASET_ID, tokenizer_id=TOKENIZER_ID,
                 selection_rate=0.15):
    """Writes a packed directory of the given ids (whole sequences of seq_len each); no device."""
    tr = np.ascontiguousarray(train, np.int32)
    ho = np.ascontiguousarray(heldout, np.int32)
    _check(lib().msx_write_packed(str(path).encode(), tr.ctypes.data, tr.size, ho.ctypes.data, ho.size, seq_len,
                                  vocabulary_size, dataset_id.encode(), tokenizer_id.encode(), selection_rate))


def check_artifact(path):
    """Validates a Hip artifact directory (no device); returns its artifact id."""
    out = ctypes.create_string_buffer(37)
    _check(lib().msx_check_artifact(str(path).encode(), out))
    return out.value.decode()


def param_shapes(step_ir):
    """[(path, shape)] of the `param` lines of a printed step, in ParamId order."""
    out = []
    for line in step_ir.splitlines():
        if line.startswith("param @"):
            path = line[len("param @"):line.index(":")]
            dims = line[line.index("[") + 1:line.index("]")]
            shape = tuple(int(d) for d in dims.split(",")) if dims.strip() else ()
            out.append((path, shape))
    return out


def param_count(step_ir):
    return int(sum(int(np.prod(s)) for _, s in param_shapes(step_ir)))


_STEPS = {"linear_regression": 500, "mnist_mlp": 1800, "mlp_classifier": 1000, "mlp_micro": 20,
          "transformer_block": 500, "block_micro": 20, "bert_tiny": 1000, "bert_cpu": 800, "bert_micro": 20,
          "bert_base": 200, "bert_micro_mixed": 20, "bert_mini_mixed": 20}


def config_steps(name):
    """The steps a config (or the .mspec file at the path `name`) trains for."""
    if name in _STEPS:
        return _STEPS[name]
    steps, seed = ctypes.c_uint64(), ctypes.c_uint64()
    L = lib()
    L.msx_config_steps.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]
    _check(L.msx_config_steps(name.encode(), ctypes.byref(steps), ctypes.byref(seed)))
    return steps.value


def bench_config(ctx, name, warmup, steps, masked_rows=-1, profile_reps=1):
    """(mean ms per step, [ms of each timed step], last loss, [(launch, ms, flop, bytes, kernels, runs)]), kernels
    the HIP kernels the launch dispatched, '+'-joined, runs how many times a profiled step ran it (a pure
    launch, such as a GEMM, is timed over back-to-back repeats)."""
    L = lib()
    L.msx_bench_config.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint32,
                                   ctypes.POINTER(ctypes.c_double), ctypes.c_void_p, ctypes.POINTER(ctypes.c_float),
                                   ctypes.c_uint32, ctypes.POINTER(ctypes.c_void_p)]
    ms, loss, rep = ctypes.c_double(), ctypes.c_float(), ctypes.c_void_p()
    per_step = np.zeros(max(1, steps), np.float64)
    _check(L.msx_bench_config(ctx._h, name.encode(), masked_rows, warmup, steps, ctypes.byref(ms),
                              per_step.ctypes.data, ctypes.byref(loss), profile_reps,
                              ctypes.byref(rep) if profile_reps else None))
    rows = []
    if profile_reps and rep.value:
        text = ctypes.string_at(rep).decode()
        L.msx_free(rep)
        for line in text.splitlines():
            what, t, flop, nbytes, kernels, runs = line.rsplit("\t", 5)
            rows.append((what, float(t), float(flop), float(nbytes), kernels, int(runs)))
    return ms.value, per_step[:steps].tolist(), loss.value, rows


def check_ir(step_ir):
    """Parse + print of a training step through the library (no device needed)."""
    out = ctypes.c_void_p()
    L = lib()
    L.msx_check_ir.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]
    _check(L.msx_check_ir(step_ir.encode(), ctypes.byref(out)))
    try:
        return ctypes.string_at(out).decode()
    finally:
        L.msx_free(out)
