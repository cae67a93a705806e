"""TEST INFRASTRUCTURE: ctypes bindings of oracle/liboracle.so, the CPU oracle (a C++
restatement of the reference interpreter). Used only as the checker of the HIP backend."""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "oracle", "liboracle.so")

vp, u64, i64, u32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int64, ctypes.c_uint32


class Oracle:
    def __init__(self):
        if not os.path.exists(LIB):
            import subprocess
            subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True)
        L = ctypes.CDLL(LIB)
        L.orc_last_error.restype = ctypes.c_char_p
        L.orc_train.argtypes = [ctypes.c_char_p, i64, i64, vp, u64, vp, u64, ctypes.POINTER(ctypes.c_double)]
        L.orc_time_steps.argtypes = [ctypes.c_char_p, i64, i64, ctypes.POINTER(ctypes.c_double)]
        L.orc_step_times.argtypes = [ctypes.c_char_p, i64, i64, vp]
        L.orc_prog_new.argtypes = [ctypes.c_char_p, ctypes.c_int, u64]
        L.orc_prog_new.restype = vp
        L.orc_prog_free.argtypes = [vp]
        L.orc_prog_run.argtypes = [vp, ctypes.c_int, vp, vp, vp, vp, ctypes.c_int, vp, vp]
        L.orc_prog_output.argtypes = [vp, ctypes.c_int, vp, u64]
        L.orc_philox.argtypes = [vp, vp, vp]
        L.orc_blake3.argtypes = [ctypes.c_char_p, u64, vp]
        L.orc_canonical_id.argtypes = [ctypes.c_char_p]
        L.orc_canonical_id.restype = u64
        L.orc_dropout_id.argtypes = [ctypes.c_char_p, u64]
        L.orc_dropout_id.restype = u64
        L.orc_dropout_threshold.argtypes = [ctypes.c_float]
        L.orc_dropout_threshold.restype = u64
        L.orc_dropout_keeps.argtypes = [u64, u64, u32, ctypes.c_float]
        L.orc_adamw_scalars.argtypes = [ctypes.c_float, u64, u64, u64, ctypes.c_float, ctypes.c_float, vp]
        L.orc_step_inputs.argtypes = [ctypes.c_char_p, i64, i64, u64, ctypes.POINTER(vp), ctypes.POINTER(vp),
                                      ctypes.POINTER(u64)]
        L.orc_free.argtypes = [vp]
        L.orc_init_params.argtypes = [ctypes.c_char_p, vp, u64]
        L.orc_train_eval.argtypes = [ctypes.c_char_p, i64, u64, u64, vp, vp, u64]
        L.orc_train_run.argtypes = [ctypes.c_char_p, ctypes.c_char_p, i64, u64, u64, vp, u64, vp, u64, vp, vp, u64]
        L.orc_corpus_draw.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int, u64, vp, vp, vp, vp, vp, vp, vp]
        L.orc_corpus_draw.restype = i64
        L.orc_uuid_of.argtypes = [vp, vp]
        L.orc_binding_id.argtypes = [ctypes.c_char_p, ctypes.c_char_p, u64, vp, vp]
        L.orc_epoch_order.argtypes = [u64, u64, u32, vp]
        L.orc_train_ckpt.argtypes = [ctypes.c_char_p, ctypes.c_char_p, i64, ctypes.c_char_p, u64, ctypes.c_char_p, vp,
                                     u64, vp, u64]
        L.orc_train_ckpt.restype = i64
        L.orc_schema_hash.argtypes = [ctypes.c_char_p, vp]
        L.orc_json_f64.argtypes = [ctypes.c_double, vp]
        L.orc_held_out_tally.argtypes = [vp, vp, vp, u64, u64, u64, vp]
        self.L = L

    def err(self):
        return self.L.orc_last_error().decode()

    def train(self, config, steps=-1, masked_rows=-1, n_params=None, n_steps=None):
        from modelspec_amd import api
        step_ir, _ = api.compile_config(config, masked_rows, steps)
        n_params = n_params or api.param_count(step_ir)
        n_steps = n_steps if n_steps is not None else (steps if steps >= 0 else api.config_steps(config))
        losses = np.zeros(n_steps + 1, np.float32)
        params = np.zeros(n_params, np.float32)
        secs = ctypes.c_double()
        rc = self.L.orc_train(config.encode(), steps, masked_rows, losses.ctypes.data, losses.size, params.ctypes.data,
                              params.size, ctypes.byref(secs))
        if rc != 0:
            raise RuntimeError(self.err())
        return losses, params, secs.value

    def train_eval(self, config, steps, eval_every, eval_batches):
        """[(step, host-finished (loss, accuracy), the oracle tally's own (loss, accuracy))]."""
        cap = steps // eval_every + 2
        at = np.zeros(cap, np.uint64)
        m = np.zeros(4 * cap, np.float32)
        n = self.L.orc_train_eval(config.encode(), steps, eval_every, eval_batches, at.ctypes.data, m.ctypes.data, cap)
        if n < 0:
            raise RuntimeError(self.err())
        return [(int(at[k]), (m[4 * k], m[4 * k + 1]), (m[4 * k + 2], m[4 * k + 3])) for k in range(n)]

    def train_packed(self, config, packed_dir, steps, eval_every=0, eval_batches=0):
        """A run on a packed directory: (losses, flat params, [(step, host (loss, acc), tally (loss, acc))])."""
        from modelspec_amd import api
        step_ir, _ = api.compile_config(config, -1, steps)
        losses = np.zeros(steps + 1, np.float32)
        params = np.zeros(api.param_count(step_ir), np.float32)
        cap = (steps // eval_every + 2) if eval_every else 1
        at = np.zeros(cap, np.uint64)
        m = np.zeros(4 * cap, np.float32)
        n = self.L.orc_train_run(config.encode(), packed_dir.encode(), steps, eval_every, eval_batches,
                                 losses.ctypes.data, losses.size, params.ctypes.data, params.size, at.ctypes.data,
                                 m.ctypes.data, cap)
        if n < 0:
            raise RuntimeError(self.err())
        evals = [(int(at[k]), (m[4 * k], m[4 * k + 1]), (m[4 * k + 2], m[4 * k + 3])) for k in range(n)]
        return losses, params, evals

    def corpus_draw(self, config, packed_dir, role, step, rows, capacity=0):
        """The CPU rows of one corpus draw: dict of ids, positions, labels, weights (and the gather's
        rows, labels, weights when capacity > 0)."""
        out = {"ids": np.zeros(rows, np.int32), "positions": np.zeros(rows, np.int32),
               "labels": np.zeros(rows, np.int32), "weights": np.zeros(rows, np.float32)}
        if capacity:
            out.update({"g_rows": np.zeros(capacity, np.int32), "g_labels": np.zeros(capacity, np.int32),
                        "g_weights": np.zeros(capacity, np.float32)})
        ptr = lambda k: out[k].ctypes.data if k in out else None
        b = self.L.orc_corpus_draw(config.encode(), packed_dir.encode(), role, step, ptr("ids"), ptr("positions"),
                                   ptr("labels"), ptr("weights"), ptr("g_rows"), ptr("g_labels"), ptr("g_weights"))
        if b < 0:
            raise RuntimeError(self.err())
        return out

    def train_ckpt(self, config, steps, packed=None, resume=None, every=0, path=None):
        """A run that may resume from a checkpoint and write checkpoints: (losses, params, start step)."""
        from modelspec_amd import api
        enc = lambda x: None if x is None else str(x).encode()
        step_ir, _ = api.compile_config(config)
        losses = np.zeros(steps + 1, np.float32)
        params = np.zeros(api.param_count(step_ir), np.float32)
        start = self.L.orc_train_ckpt(config.encode(), enc(packed), steps, enc(resume), every, enc(path),
                                      losses.ctypes.data, losses.size, params.ctypes.data, params.size)
        if start < 0:
            raise RuntimeError(self.err())
        return losses, params, start

    def schema_hash(self, config):
        buf = ctypes.create_string_buffer(65)
        if self.L.orc_schema_hash(config.encode(), buf) != 0:
            raise RuntimeError(self.err())
        return buf.value.decode()

    def json_f64(self, v):
        buf = ctypes.create_string_buffer(40)
        self.L.orc_json_f64(v, buf)
        return buf.value.decode()

    def uuid_of(self, digest):
        buf = ctypes.create_string_buffer(37)
        d = (ctypes.c_uint8 * 32)(*digest)
        self.L.orc_uuid_of(d, buf)
        return buf.value.decode()

    def binding_id(self, dataset_id, tokenizer_id, seq_len, rates):
        buf = ctypes.create_string_buffer(37)
        r = np.array(rates, np.float64)
        if self.L.orc_binding_id(dataset_id.encode(), tokenizer_id.encode(), seq_len, r.ctypes.data, buf) != 0:
            return None
        return buf.value.decode()

    def epoch_order(self, seed, epoch, n):
        out = np.zeros(n, np.uint32)
        self.L.orc_epoch_order(seed, epoch, n, out.ctypes.data)
        return out

    def held_out_tally(self, logits, labels, weights):
        """logits [batches, rows, v] f32, labels [batches, rows] i32, weights [batches, rows] f32 ->
        dict(loss, accuracy, numerator, denominator, correct, selected), the eval.rs tally."""
        logits = np.ascontiguousarray(logits, np.float32)
        labels = np.ascontiguousarray(labels, np.int32)
        weights = np.ascontiguousarray(weights, np.float32)
        b, r, v = logits.shape
        out = np.zeros(6, np.float64)
        if self.L.orc_held_out_tally(logits.ctypes.data, labels.ctypes.data, weights.ctypes.data, b, r, v,
                                     out.ctypes.data) != 0:
            raise ValueError(self.err())
        keys = ("loss", "accuracy", "numerator", "denominator", "correct", "selected")
        return {k: (np.float32(x) if k in ("loss", "accuracy") else x) for k, x in zip(keys, out)}

    def seconds_per_step(self, config, steps, masked_rows=-1):
        s = ctypes.c_double()
        if self.L.orc_time_steps(config.encode(), steps, masked_rows, ctypes.byref(s)) != 0:
            raise RuntimeError(self.err())
        return s.value

    def step_times(self, config, steps, masked_rows=-1):
        """Seconds of each of `steps` training steps from the initial parameters, one thread."""
        out = np.zeros(steps, np.float64)
        if self.L.orc_step_times(config.encode(), steps, masked_rows, out.ctypes.data) != 0:
            raise RuntimeError(self.err())
        return out

    def philox(self, counter, key):
        c = np.array(counter, np.uint32)
        k = np.array(key, np.uint32)
        o = np.zeros(4, np.uint32)
        self.L.orc_philox(c.ctypes.data, k.ctypes.data, o.ctypes.data)
        return [int(x) for x in o]

    def blake3(self, data):
        out = (ctypes.c_uint8 * 32)()
        self.L.orc_blake3(data, len(data), out)
        return bytes(out)

    def canonical_id(self, path):
        return self.L.orc_canonical_id(path.encode())

    def dropout_id(self, site, step):
        return self.L.orc_dropout_id(site.encode(), step)

    def dropout_threshold(self, p):
        return self.L.orc_dropout_threshold(p)

    def dropout_keeps(self, seed, id_, index, p):
        return bool(self.L.orc_dropout_keeps(seed, id_, index, p))

    def adamw_scalars(self, lr, t, steps, warmup, beta1=0.9, beta2=0.999):
        o = np.zeros(3, np.float32)
        self.L.orc_adamw_scalars(lr, t, steps, warmup, beta1, beta2, o.ctypes.data)
        return o

    def step_inputs(self, config, step, steps=-1, masked_rows=-1):
        names, data, words = vp(), vp(), u64()
        if self.L.orc_step_inputs(config.encode(), steps, masked_rows, step, ctypes.byref(names), ctypes.byref(data),
                                  ctypes.byref(words)) != 0:
            raise RuntimeError(self.err())
        text = ctypes.string_at(names).decode()
        raw = np.frombuffer(ctypes.string_at(data, words.value * 4), np.uint32).copy()
        self.L.orc_free(names)
        self.L.orc_free(data)
        out, off = {}, 0
        for line in text.splitlines():
            name, dt, n = line.split("\t")
            n = int(n)
            chunk = raw[off:off + n]
            off += n
            out[name] = chunk.view(np.float32) if dt == "f32" else chunk.view(np.int32)
        return out

    def init_params(self, config, n):
        out = np.zeros(n, np.float32)
        if self.L.orc_init_params(config.encode(), out.ctypes.data, n) != 0:
            raise RuntimeError(self.err())
        return out

    def run_program(self, text, inputs, params=(), seed=0, outputs=(0,)):
        """Evaluates a printed program; returns the requested outputs as float32 arrays."""
        h = self.L.orc_prog_new(text.encode(), 1, seed)
        if not h:
            raise RuntimeError(self.err())
        try:
            names = [n.encode() for n in inputs]
            arrs = [np.ascontiguousarray(a) for a in inputs.values()]
            n = len(arrs)
            c_names = (ctypes.c_char_p * max(1, n))(*names)
            c_dt = (ctypes.c_int * max(1, n))(*[0 if a.dtype == np.float32 else 1 for a in arrs])
            c_data = (ctypes.c_void_p * max(1, n))(*[a.ctypes.data for a in arrs])
            c_cnt = (ctypes.c_uint64 * max(1, n))(*[a.size for a in arrs])
            ps = [np.ascontiguousarray(p, np.float32) for p in params]
            c_p = (ctypes.c_void_p * max(1, len(ps)))(*[p.ctypes.data for p in ps])
            c_pc = (ctypes.c_uint64 * max(1, len(ps)))(*[p.size for p in ps])
            if self.L.orc_prog_run(h, n, c_names, c_dt, c_data, c_cnt, len(ps), c_p, c_pc) != 0:
                raise RuntimeError(self.err())
            res = []
            for k in outputs:
                cnt = output_count(text, k)
                o = np.zeros(cnt, np.float32)
                if self.L.orc_prog_output(h, k, o.ctypes.data, cnt) != 0:
                    raise RuntimeError(self.err())
                res.append(o)
            return res
        finally:
            self.L.orc_prog_free(h)


def output_count(text, k):
    """Element count of output k of a printed program."""
    outs = [int(line.split("%")[1].split()[0]) for line in text.splitlines() if line.startswith("output %")]
    want = outs[k]
    for line in text.splitlines():
        s = line
        for tag in ("forward ", "loss ", "gradient ", "optimizer "):
            if s.startswith(tag):
                s = s[len(tag):]
        if s.startswith(f"%{want}:"):
            dims = s[s.index("[") + 1:s.index("]")]
            return int(np.prod([int(d) for d in dims.split(",")])) if dims.strip() else 1
    raise KeyError(want)
