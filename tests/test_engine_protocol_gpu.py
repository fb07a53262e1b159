"""kiln_engine (kiln_amd/host/engine_main.cpp): the engine process of the JSON-lines protocol (the reference's
engine/src/main.cpp:620-801 and parse_job :562-600, Engine::generate engine.h:672-792), checked against the
request and event format that the reference's fake backend server/mock-engine.js and README.md:399-434 define:
ready first; per generate job encoded -> step (stage, step, of, ms, preview {w, h, rgb base64 RGB8 at latent
size}) x steps -> decoded -> done (out, w, h, total_ms, timings), the output file raw RGB8 [h, w, 3]; cancel of a
queued job and of a running one; error events for bad jobs and for commands this build does not run; info.
The DiT is small (2 blocks, 4 heads) so the test takes seconds."""
import base64
import json
import os
import subprocess
import time

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ENGINE = os.path.join(ROOT, "kiln_amd", "kiln_engine")

# event name -> keys every such event carries (server/mock-engine.js, README.md:421-434)
SCHEMA = {
    "ready": {"ev"}, "log": {"ev", "msg"}, "loading": {"ev", "what"}, "info": {"id", "ev", "gpu"},
    "encoded": {"id", "ev", "ms"}, "step": {"id", "ev", "stage", "step", "of", "ms"}, "decoded": {"id", "ev", "ms"},
    "done": {"id", "ev"}, "error": {"id", "ev", "msg"}, "cancelled": {"id", "ev"},
}


def _job(jid, out, **kw):
    r = dict(cmd="generate", id=jid, width=128, height=96, steps=3, cfg=1, sampler="euler", scheduler="simple",
             shift=3, seed=777, qwen_ids=[9707, 11, 1879], t5_ids=[1], t5_weights=[1.0],
             neg={"qwen_ids": [3, 4], "t5_ids": [1]}, nag={"enabled": True, "scale": 5, "tau": 2.5, "alpha": 0.25},
             out=out)
    r.update(kw)
    return json.dumps(r)


class Engine:
    def __init__(self, errfile):
        self.err = open(errfile, "w+")
        self.p = subprocess.Popen([ENGINE, "--blocks", "2", "--heads", "4"], stdin=subprocess.PIPE,
                                  stdout=subprocess.PIPE, stderr=self.err, text=True, bufsize=1)
        self.events = []

    def send(self, line):
        self.p.stdin.write(line + "\n")
        self.p.stdin.flush()

    def read_until(self, pred, timeout=60):
        t0 = time.time()
        while time.time() - t0 < timeout:
            line = self.p.stdout.readline()
            if not line:
                break
            e = json.loads(line)
            self.events.append(e)
            if pred(e):
                return e
        raise AssertionError(f"no matching event; last events: {self.events[-5:]}")

    def close(self, timeout=120):
        """Closes stdin (the engine finishes its queue and exits) and reads the remaining events."""
        self.p.stdin.close()
        out = self.p.stdout.read()
        rc = self.p.wait(timeout=timeout)
        self.events += [json.loads(ln) for ln in out.splitlines() if ln.strip()]
        self.err.seek(0)
        return rc, self.err.read()


@pytest.fixture(scope="module")
def session(tmp_path_factory):
    assert os.path.exists(ENGINE), "kiln_engine is not built (python -m kiln_amd.build)"
    d = tmp_path_factory.mktemp("engine")
    e = Engine(d / "engine.err")
    ready = e.read_until(lambda ev: ev["ev"] in ("ready", "fatal"))
    assert ready["ev"] == "ready", ready
    # a long job, cancelled while it runs (after its first step)
    e.send(_job("long", str(d / "long.rgb"), steps=40))
    e.read_until(lambda ev: ev.get("id") == "long" and ev["ev"] == "step")
    e.send(json.dumps({"cmd": "cancel", "id": "long"}))
    e.read_until(lambda ev: ev.get("id") == "long" and ev["ev"] in ("cancelled", "done", "error"))
    e.send(json.dumps({"cmd": "info", "id": "i1"}))
    e.send(_job("j1", str(d / "j1.rgb")))
    e.send(_job("j2", str(d / "j2.rgb")))  # the same job: the same image
    e.send(_job("j3", str(d / "j3.rgb"), cfg=4.5, seed=778, preview=False, sampler="dpmpp_2m", scheduler="karras",
                steps=6, step_cache=0.1))
    e.send(_job("j4", str(d / "j4.rgb")))
    e.send(json.dumps({"cmd": "cancel", "id": "j4"}))  # still queued behind j1..j3
    e.send("this is not json")
    e.send(json.dumps({"cmd": "graph", "id": "g1", "nodes": {}}))
    e.send(_job("j5", "", width=100))  # no out path
    e.send(_job("j6", "", skip_decode=True, sampler="er_sde", steps=3))
    e.send(_job("j7", str(d / "j7.rgb"), family="sdxl"))
    rc, err = e.close()
    assert rc == 0, err[-2000:]
    return e.events, d


def _of(events, jid):
    return [e for e in events if e.get("id") == jid]


def test_every_event_is_well_formed(session):
    events, _ = session
    assert events[0]["ev"] in ("log", "loading", "ready")
    first_ready = next(i for i, e in enumerate(events) if e["ev"] == "ready")
    assert all("id" not in e or e["id"] == "" for e in events[:first_ready])
    for e in events:
        assert e["ev"] in SCHEMA, e
        missing = SCHEMA[e["ev"]] - set(e)
        assert not missing, (e, missing)
    assert any(e["ev"] == "log" and "bad request" in e["msg"] for e in events)


def test_generate_event_sequence_and_output(session):
    events, d = session
    ev = _of(events, "j1")
    names = [e["ev"] for e in ev]
    assert names == ["encoded", "step", "step", "step", "decoded", "done"], names
    steps = [e for e in ev if e["ev"] == "step"]
    assert [s["step"] for s in steps] == [1, 2, 3] and all(s["of"] == 3 and s["stage"] == "base" for s in steps)
    for s in steps:
        p = s["preview"]
        assert (p["w"], p["h"]) == (128 // 8, 96 // 8)
        assert len(base64.b64decode(p["rgb"])) == p["w"] * p["h"] * 3
        assert isinstance(s["ms"], int) and s["ms"] >= 0
    done = ev[-1]
    assert done["out"] == str(d / "j1.rgb") and (done["w"], done["h"]) == (128, 96)
    assert isinstance(done["total_ms"], int)
    for k in ("encode_ms", "sample_ms", "decode_ms"):
        assert isinstance(done["timings"][k], int)
    img = (d / "j1.rgb").read_bytes()
    assert len(img) == 128 * 96 * 3 and len(set(img)) > 16  # an image, not a constant


def test_same_job_same_image_other_seed_other_image(session):
    _, d = session
    assert (d / "j1.rgb").read_bytes() == (d / "j2.rgb").read_bytes()
    assert (d / "j1.rgb").read_bytes() != (d / "j3.rgb").read_bytes()


def test_cfg_sampler_scheduler_cache_and_preview_off(session):
    events, d = session
    ev = _of(events, "j3")
    steps = [e for e in ev if e["ev"] == "step"]
    assert len(steps) == 6 and all("preview" not in s for s in steps)
    done = ev[-1]
    assert done["ev"] == "done" and "cache_skips" in done["timings"]
    assert len((d / "j3.rgb").read_bytes()) == 128 * 96 * 3


def test_cancel_queued_and_running(session):
    events, _ = session
    assert [e["ev"] for e in _of(events, "j4")] == ["cancelled"]
    long = _of(events, "long")
    assert long[-1]["ev"] == "cancelled"
    assert 1 <= sum(e["ev"] == "step" for e in long) < 40


def test_errors_and_unsupported(session):
    events, _ = session
    g = _of(events, "g1")
    assert [e["ev"] for e in g] == ["error"] and "not supported" in g[0]["msg"]
    j5 = _of(events, "j5")
    assert j5[-1]["ev"] == "error" and "out path" in j5[-1]["msg"]
    j6 = _of(events, "j6")
    assert j6[-1]["ev"] == "done" and j6[-1].get("skipped_decode") is True
    assert sum(e["ev"] == "step" for e in j6) == 3
    j7 = _of(events, "j7")
    assert [e["ev"] for e in j7] == ["error"]


def test_info(session):
    events, _ = session
    info = _of(events, "i1")
    assert len(info) == 1 and info[0]["ev"] == "info" and info[0]["vram_free_mb"] > 0
