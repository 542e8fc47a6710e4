"""Reading and setting torch's current stream on the host path of `Cohort.sample`.

torch's public calls for this, `torch.cuda.current_stream` and `torch.cuda.set_stream`, build a `torch.cuda.Stream`
object on every call, and `sample` switches streams several times per call. The bindings those public calls are built
on, `torch._C._cuda_getCurrentStream(device)` and `torch._C._cuda_setStream(stream_id, device_index, device_type)`,
take and return the plain (stream id, device index, device type) triple instead. They are private, so this module
uses them only on torch versions they were checked against (`CHECKED`) and only after a first call has shown that
they agree with the public calls on this process's device (`verify`); otherwise, and for any other torch, it uses the
public calls. Both give the same stream triples.
"""
import torch

CHECKED = ("2.10.",)          # torch versions whose private bindings were checked (tests/test_host.py, tests/test_gpu_sampler.py)


def _public_get(device_index):
    s = torch.cuda.current_stream(device_index)
    return (s.stream_id, s.device_index, s.device_type)


def _public_set(stream_id, device_index, device_type):
    torch.cuda.set_stream(torch.cuda.Stream(stream_id=stream_id, device_index=device_index, device_type=device_type))


class StreamOps:
    """get(device_index) -> the current stream's triple; set(stream_id, device_index, device_type) makes that stream
    current."""

    def __init__(self, version=None, module=None):
        version = torch.__version__ if version is None else version
        module = torch._C if module is None else module
        g, s = getattr(module, "_cuda_getCurrentStream", None), getattr(module, "_cuda_setStream", None)
        self.private = bool(g and s and any(version.startswith(v) for v in CHECKED))
        self._checked, self._g, self._s = not self.private, g, s
        self.get, self.set = (g, s) if self.private else (_public_get, _public_set)
        if self.private:
            self.get, self.set = self._first_get, self._first_set

    def _first_get(self, device_index):
        self.verify(device_index)
        return self.get(device_index)

    def _first_set(self, stream_id, device_index, device_type):
        self.verify(device_index)
        return self.set(stream_id, device_index, device_type)

    def verify(self, device_index):
        """On first use: the private bindings must read the public calls' triple and set a stream the public calls then
        report; else the public calls from here on."""
        if self._checked:
            return
        self._checked = True
        g, s = self._g, self._s
        ok = False
        before = _public_get(device_index)
        try:
            t = g(device_index)
            if tuple(t) == before:
                other = torch.cuda.Stream(device=device_index)
                s(other.stream_id, other.device_index, other.device_type)
                ok = _public_get(device_index) == (other.stream_id, other.device_index, other.device_type)
        except (TypeError, RuntimeError, AttributeError):
            ok = False
        finally:
            _public_set(*before)
        if ok:
            self.get, self.set = g, s
        else:
            self.private = False
            self.get, self.set = _public_get, _public_set


ops = StreamOps()
