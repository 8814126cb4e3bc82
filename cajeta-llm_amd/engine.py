"""The LlmEngine surface over the MI355X backend.

Mirrors the reference's host API for the decode path — LlmEngine.load /
submitTokens / runAll / stepOnce / request / cancel / close / eogTokens
(L/LlmEngine.cajeta:165-546), EngineOptions (L/EngineOptions.cajeta:10-122),
SampleParams (L/gen/SampleParams.cajeta:25-43) and the KernelCap registry
(L/model/KernelCap.cajeta:228-300) — with the same names and error
behaviour (LlmException). Here L/ is src/main/cajeta/dev/cajeta/llm/.
"""
import ctypes

import numpy as np

from . import native
from .native import LlmException, check, handle, lib, ptr


class EngineOptions:
    """Options for LlmEngine.load (the decode-relevant EngineOptions fields)."""

    def __init__(self, model):
        self.model = "" + model
        self.ctx = 4096
        self.maxSeqs = 4
        self.device = ""
        self.cpuThreads = 0      # the CPU worker count the attention split rule follows (0: 512)
        self.graphs = True       # replay the captured decode step (False: eager launches)
        self.prefillChunk = 512  # rows a prefill chunk (CausalLM.CHUNK_MAX); 0: one decode step a position
        self.kvBlocks = 0        # K/V pool pages of 64 positions shared by the slots (0: every slot at full context;
                                 # CausalLM's numBlocks): a smaller pool preempts under pressure
        self.kvF32 = False       # f32 K/V planes (PagedKvCache's mode; the two-pass attention models)


class SampleParams:
    """Greedy only: temperature 0 and no penalty (Sampler.isGreedy,
    L/gen/Sampler.cajeta:41-46); anything else is refused by name."""

    def __init__(self, temperature=0.0, topK=0, topP=1.0, repeatPenalty=1.0, stopTokens=None):
        self.temperature = temperature
        self.topK = topK
        self.topP = topP
        self.repeatPenalty = repeatPenalty
        self.stopTokens = list(stopTokens) if stopTokens else None

    def isGreedy(self):
        return self.temperature == 0.0 and self.repeatPenalty == 1.0


class Request:
    """A request's state as the scheduler left it (sched/Request.cajeta)."""
    WAITING, RUNNING, PREEMPTED, DONE = 0, 1, 2, 3
    FINISH_NONE, FINISH_BUDGET, FINISH_EOS, FINISH_CANCEL = 0, 1, 2, 4

    def __init__(self, rid, tokens, state, reason):
        self.id = rid
        self.tokens = tokens
        self.state = state
        self.done = state == Request.DONE
        self.finishReason = reason

    def generatedCount(self):
        return len(self.tokens)

    def generatedAt(self, i):
        return self.tokens[i]


class KernelCap:
    """Which kernels this backend registered, asked of the library's registry
    under the reference's kernel names; overrides as the reference's
    setOverride/clearOverrides (L/model/KernelCap.cajeta:272-300)."""

    _overrides = {}

    @staticmethod
    def usable(name):
        if name in KernelCap._overrides:
            return KernelCap._overrides[name]
        native.init()
        return lib().cj_kernel_available(name.encode()) == 1

    @staticmethod
    def setOverride(name, on):
        KernelCap._overrides[name] = bool(on)

    @staticmethod
    def clearOverrides():
        KernelCap._overrides.clear()


class LlmEngine:
    """load -> submitTokens -> runAll -> request(id), over one GGUF model."""

    def __init__(self, h, opts):
        self.h = h
        self.opts = opts
        cfg = (ctypes.c_int64 * 14)()
        check(lib().cj_engine_config(h, cfg, 14), "cj_engine_config")
        keys = ("numLayers", "hiddenSize", "numHeads", "numKvHeads", "headDim", "intermediateSize", "vocabSize",
                "ctx", "expertCount", "expertUsedCount", "weightType", "headType", "expertFfn", "attnWorkers")
        self.config = dict(zip(keys, [int(v) for v in cfg]))
        self._eog = []
        self._batch_rows = 0

    @staticmethod
    def load(opts):
        if isinstance(opts, str):
            opts = EngineOptions(opts)
        dev = 0
        if opts.device not in ("", "hip", "gpu", "rocm"):
            if opts.device.startswith("hip:"):
                dev = int(opts.device[4:])
            else:
                raise LlmException("engine: device '%s' is not served by the MI355X backend" % opts.device)
        native.init(dev)
        h = lib().cj_engine_load_kv(opts.model.encode(), int(opts.ctx), int(opts.maxSeqs),
                                    int(getattr(opts, "kvBlocks", 0)), int(bool(getattr(opts, "kvF32", False))))
        handle(h, "LlmEngine.load(%s)" % opts.model)
        if not getattr(opts, "graphs", True):
            check(lib().cj_engine_set_graphs(h, 0), "cj_engine_set_graphs")
        if getattr(opts, "cpuThreads", 0):
            check(lib().cj_engine_set_cpu_threads(h, int(opts.cpuThreads)), "cj_engine_set_cpu_threads")
        chunk = getattr(opts, "prefillChunk", 512)
        if chunk != 512:
            check(lib().cj_engine_set_prefill_chunk(h, int(chunk)), "cj_engine_set_prefill_chunk")
        return LlmEngine(h, opts)

    # -- the LlmEngine surface
    def submitTokens(self, prompt, promptLen=None, maxNew=16, params=None):
        params = params or SampleParams()
        if not params.isGreedy():
            raise LlmException("engine: the MI355X decode path serves greedy sampling only")
        p = np.ascontiguousarray(prompt[: promptLen if promptLen is not None else len(prompt)], dtype=np.int32)
        if params.stopTokens is None:   # LlmEngine.defaultStops: the model's EOG set
            return check(lib().cj_engine_submit(self.h, ptr(p), int(p.size), int(maxNew)), "submitTokens")
        st = np.ascontiguousarray(params.stopTokens, dtype=np.int32)
        return check(lib().cj_engine_submit_stops(self.h, ptr(p), int(p.size), int(maxNew), ptr(st), int(st.size)),
                     "submitTokens")

    def submitText(self, prompt, params=None, maxNew=16):
        raise LlmException("engine: no tokenizer - load a GGUF or submit token ids")

    def runAll(self, maxSteps=1 << 20):
        """Step until every request is done; raises past maxSteps (Scheduler.runAll)."""
        check(lib().cj_engine_run_all(self.h, int(maxSteps)), "runAll")

    def stepOnce(self):
        """One scheduler step; True while a request is unfinished."""
        return check(lib().cj_engine_step_once(self.h), "stepOnce") == 1

    def request(self, rid):
        cap = 1 << 16
        out = np.zeros(cap, np.int32)
        state = ctypes.c_int32(0)
        reason = ctypes.c_int32(0)
        n = check(lib().cj_engine_request(self.h, int(rid), ptr(out), cap, ctypes.byref(state), ctypes.byref(reason)),
                  "request")
        return Request(rid, out[:n].tolist(), int(state.value), int(reason.value))

    def cancel(self, rid):
        return check(lib().cj_engine_cancel(self.h, int(rid)), "cancel") == 1

    def textOf(self, rid):
        raise LlmException("engine: no tokenizer for detok")

    def eogTokens(self):
        return list(self._eog)

    def setEog(self, ids):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        self._eog = a.tolist()
        check(lib().cj_engine_set_eog(self.h, ptr(a), int(a.size)), "setEog")

    def close(self):
        if self.h:
            lib().cj_engine_close(self.h)
            self.h = 0

    # -- the CausalLM seam (model/CausalLM.cajeta:801-1256)
    def reset(self, seq=0):
        check(lib().cj_engine_reset(self.h, seq), "reset")

    def prefill(self, tokens, seq=0):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        check(lib().cj_engine_prefill(self.h, seq, ptr(t), int(t.size)), "prefill")

    def decode(self, steps, seq=0):
        out = np.zeros(max(1, steps), np.int32)
        check(lib().cj_engine_decode(self.h, seq, int(steps), ptr(out)), "decode")
        return out[:steps]

    def decodeBatch(self, seqs, steps):
        """`steps` greedy tokens for each prefilled slot in `seqs` at once
        (CausalLM.decodeBatchRows): an int32 array [steps][len(seqs)]."""
        sl = np.ascontiguousarray(seqs, dtype=np.int32)
        out = np.zeros((max(1, steps), sl.size), np.int32)
        check(lib().cj_engine_decode_batch(self.h, ptr(sl), int(sl.size), int(steps), ptr(out)), "decodeBatch")
        self._batch_rows = int(sl.size)
        return out[:steps]

    def batchLogits(self):
        """The last batched decode step's logits, [rows][vocab]."""
        v = self.config["vocabSize"]
        rows = self._batch_rows
        out = np.empty(rows * v, np.float32)
        check(lib().cj_engine_trace(self.h, 6, ptr(out), out.size), "batchLogits")
        return out.reshape(rows, v)

    def logits(self, seq=0):
        out = np.empty(self.config["vocabSize"], np.float32)
        check(lib().cj_engine_logits(self.h, seq, ptr(out), out.size), "logits")
        return out

    def preds(self, n, seq=0):
        out = np.empty(n, np.int32)
        check(lib().cj_engine_preds(self.h, seq, ptr(out), int(n)), "preds")
        return out

    def trace(self, what):
        """The last step's buffer `what` (0 hs, 1 q, 2 attn, 3 act, 4 logits)."""
        c = self.config
        n = {0: c["hiddenSize"], 1: c["numHeads"] * c["headDim"], 2: c["numHeads"] * c["headDim"],
             3: c["intermediateSize"], 4: c["vocabSize"]}[what]
        out = np.empty(n, np.float32)
        check(lib().cj_engine_trace(self.h, int(what), ptr(out), n), "trace")
        return out

    def lastStepMicros(self):
        return float(lib().cj_engine_last_step_us(self.h))

    def timeKernel(self, kind, reps=100, seq=0):
        """Mean µs of `reps` eager launches of one launch kind of the step
        (layer 0), its algorithmic HBM bytes and its kernel name."""
        us = np.zeros(1, np.float32)
        nb = np.zeros(1, np.int64)
        name = np.zeros(128, np.int8)
        check(lib().cj_engine_time_kernel(self.h, seq, int(kind), int(reps), ptr(us), ptr(nb), ptr(name), 128),
              "time kernel")
        return float(us[0]), int(nb[0]), bytes(name.view(np.uint8)).split(b"\0")[0].decode()

    def timeKernelInStep(self, kind, steps=4, seq=0):
        """Mean µs of one launch kind inside whole eager decode steps (every
        layer's launch, an event before and after each)."""
        us = np.zeros(1, np.float32)
        check(lib().cj_engine_time_kernel_in_step(self.h, seq, int(kind), int(steps), ptr(us)), "time kernel in step")
        return float(us[0])

    def stepBytes(self, count):
        """Algorithmic HBM bytes of one decode step attending `count` positions."""
        v = int(lib().cj_engine_step_bytes(self.h, int(count)))
        if v < 0:
            check(v, "step bytes")
        return v

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def synth_gguf(spec, path, seed=0):
    """A seeded random-init GGUF for a config ("c1".."c5" or key=value;...),
    written to `path` or to an in-process image ("mem:<name>")."""
    check(lib().cj_synth_gguf(spec.encode(), path.encode(), int(seed)), "synth_gguf(%s)" % spec)
    return path


def image_bytes(name):
    """A read-only numpy view of an in-process image (for checkers)."""
    addr = ctypes.c_int64(0)
    size = ctypes.c_int64(0)
    check(lib().cj_image_info(name.encode(), ctypes.byref(addr), ctypes.byref(size)), "image_info")
    buf = (ctypes.c_uint8 * size.value).from_address(addr.value)
    return np.frombuffer(buf, dtype=np.uint8)


def image_free(name):
    check(lib().cj_image_free(name.encode()), "image_free")
