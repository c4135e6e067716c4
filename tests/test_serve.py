"""The /v1/systemone application and CLI on the CPU, with stand-in deciders (no GPU): routing, status
codes, limits, budgets, model selection and the answer decorations, as the reference's server
answers them (src/deciax/serve/app.py, src/deciax/protocol/systemone.py)."""

from __future__ import annotations

import http.client
import json
import threading
import time
from typing import Any

import pytest

from deciax_amd.serve import contract
from deciax_amd.serve.wsgi import DecisionApp, make_server

QUESTIONS = {"mood": {"type": "choice", "criteria": {"pos": "positive", "neg": "negative"}},
             "urgent": {"type": "noul"}}


class Model:
    max_token_budget = 4096


class FakeDecider:
    """Answers with fixed probabilities; records the budgets it was called with."""

    def __init__(self, name: str = "tiny", fail: BaseException | None = None) -> None:
        self.name, self.fail, self.model, self.calls = name, fail, Model(), []

    def _answer(self, state: Any) -> dict[str, Any]:
        if self.fail is not None:
            raise self.fail
        return {"model": self.name, "usage": {"input_tokens": len(str(state)), "output_tokens": 0},
                "answers": {"mood": {"type": "choice", "choice": "pos", "confidence": 0.75,
                                     "probabilities": {"pos": 0.75, "neg": 0.25}},
                            "urgent": {"type": "noul", "noul": 0.1}}}

    def decide(self, state, questions, **budgets):
        self.calls.append(budgets)
        return self._answer(state)

    def decide_batch(self, states, questions, **budgets):
        self.calls.append(budgets)
        return [self._answer(s) for s in states]


def post(service: DecisionApp, path: str, body: Any, headers: dict[str, str] | None = None):
    raw = body if isinstance(body, bytes) else json.dumps(body).encode()
    return service.respond("POST", path, headers or {}, raw)


def test_routes_methods_and_health() -> None:
    s = DecisionApp({"tiny": FakeDecider()}, "tiny", api_key="k", device="gfx950")
    assert s.respond("GET", "/nope", {}, b"").status == 404
    assert s.respond("GET", "/v1/systemone", {}, b"").status == 405
    assert s.respond("POST", "/health", {}, b"").status == 405
    assert s.respond("GET", "/health", {}, b"").payload == {"status": "ok"}
    full = s.respond("GET", "/health/", {"authorization": "Bearer k"}, b"").payload
    assert full == {"status": "ok", "loaded": ["tiny"], "default_model": "tiny", "device": "gfx950"}
    assert post(s, "/v1/systemone", {"state": "x", "questions": QUESTIONS}).status == 401
    ok = post(s, "/v1/systemone?x=1", {"state": "x", "questions": QUESTIONS}, {"authorization": "Bearer k"})
    assert ok.status == 200 and "Server-Timing" in ok.headers and "X-Inference-Time-Ms" in ok.headers


def test_answers_carry_jev_confidence_or_the_strict_view() -> None:
    r = post(DecisionApp({"tiny": FakeDecider()}, "tiny"), "/v1/systemone", {"state": "x", "questions": QUESTIONS})
    mood = r.payload["answers"]["mood"]
    assert mood["x_jev_confidence"] == 0.5  # (0.75 - 1/2) / (1 - 1/2)
    assert "x_jev_confidence" not in r.payload["answers"]["urgent"]
    strict = post(DecisionApp({"tiny": FakeDecider()}, "tiny", jev_strict=True), "/v1/systemone",
                  {"state": "x", "questions": QUESTIONS}).payload
    assert set(strict["answers"]["mood"]) == {"type", "choice", "confidence", "probabilities"}
    assert strict["usage"] == {"input_tokens": 1, "output_tokens": 0}
    batch = post(DecisionApp({"tiny": FakeDecider()}, "tiny"), "/v1/systemone/batch",
                 {"states": ["ab", "cde"], "questions": QUESTIONS}).payload
    assert len(batch["results"]) == 2 and batch["total_usage"] == {"input_tokens": 5, "output_tokens": 0}


def test_jev_confidence_kats() -> None:
    c = contract.confidence
    assert c({"type": "choice", "probabilities": {"a": 1.0, "b": 0.0}}) == 1.0
    assert c({"type": "choice", "probabilities": {"a": 0.5, "b": 0.5}}) == 0.0
    assert c({"type": "choice", "probabilities": {"a": 1.0}}) == 1.0
    assert c({"type": "score", "probabilities": {"0": 0.0, "1": 1.0, "2": 0.0}}) == 1.0
    # uniform over 3 levels: spread from the mode (level 0) is 1, the uniform spread 2/3 -> clamped to 0
    assert c({"type": "score", "probabilities": {"0": 1 / 3, "1": 1 / 3, "2": 1 / 3}}) == 0.0
    assert c({"type": "noul", "noul": 0.3}) is None
    assert c({"type": "choice", "probabilities": {"a": True}}) is None
    assert c({"type": "choice", "probabilities": {"a": float("nan"), "b": 1.0}}) is None


@pytest.mark.parametrize("body,status", [
    (b"{not json", 400),
    ({"state": "x"}, 400),
    ({"questions": QUESTIONS}, 400),                                               # state missing
    ({"state": "x", "questions": []}, 400),
    ({"state": "x", "questions": {f"q{i}": {"type": "noul"} for i in range(65)}}, 413),
    ({"state": "x", "questions": {"c": {"type": "choice", "criteria": {str(i): "o" for i in range(101)}}}}, 413),
    ({"state": "x", "questions": {"s": {"type": "score", "criteria": ["a", None]}}}, 422),
    ({"state": "x" * 50001, "questions": QUESTIONS}, 413),
    ({"state": "x", "questions": QUESTIONS, "lang": "en"}, 422),
    ({"state": "x", "questions": QUESTIONS, "hooks": []}, 422),
    ({"state": "\ud800", "questions": QUESTIONS}, 400),
    ({"state": "x", "questions": QUESTIONS, "max_len": True}, 422),
    ({"state": "x", "questions": QUESTIONS, "max_len": 0}, 422),
    ({"state": "x", "questions": QUESTIONS, "max_len": 4097}, 422),
    ({"state": "x", "questions": QUESTIONS, "model": "gemma2-27b"}, 422),           # registered, not loaded
    ({"state": "x", "questions": QUESTIONS, "model": "../weights"}, 422),
])
def test_client_errors(body: Any, status: int) -> None:
    r = post(DecisionApp({"tiny": FakeDecider()}, "tiny"), "/v1/systemone", body)
    assert r.status == status, r.payload
    assert isinstance(r.payload["detail"], str)


def test_batch_limits_and_body_size() -> None:
    s = DecisionApp({"tiny": FakeDecider()}, "tiny")
    assert post(s, "/v1/systemone/batch", {"states": [], "questions": QUESTIONS}).status == 400
    assert post(s, "/v1/systemone/batch", {"states": ["x"] * 65, "questions": QUESTIONS}).status == 413
    assert post(s, "/v1/systemone/batch", {"states": ["x"], "questions": QUESTIONS, "batch_size": 4}).status == 422
    assert post(s, "/v1/systemone", b" " * (contract.MAX_BODY_BYTES + 1)).status == 413


def test_budgets_and_model_selection() -> None:
    a, b = FakeDecider("tiny"), FakeDecider("other")
    s = DecisionApp({"tiny": a, "other": b}, "tiny")
    assert post(s, "/v1/systemone", {"state": "x", "questions": QUESTIONS, "max_len": 100}).status == 200
    assert a.calls[-1] == {"max_len": 100}
    post(s, "/v1/systemone", {"state": "x", "questions": QUESTIONS, "model": "other"})
    assert len(b.calls) == 1
    post(s, "/v1/systemone", {"state": "x", "questions": QUESTIONS, "model": "jev-1"})  # unknown: server's choice
    assert len(a.calls) == 2


def test_model_errors_map_to_422_and_500() -> None:
    bad = DecisionApp({"tiny": FakeDecider(fail=ValueError("schema requires 9999 tokens"))}, "tiny")
    r = post(bad, "/v1/systemone", {"state": "x", "questions": QUESTIONS})
    assert r.status == 422 and "9999" in r.payload["detail"]
    broken = DecisionApp({"tiny": FakeDecider(fail=RuntimeError("device lost"))}, "tiny")
    r = post(broken, "/v1/systemone", {"state": "x", "questions": QUESTIONS})
    assert r.status == 500 and r.payload == {"detail": "inference failed"}


def test_admission_limit_returns_503() -> None:
    gate, entered = threading.Event(), threading.Event()

    class Slow(FakeDecider):
        def decide(self, state, questions, **budgets):
            entered.set()
            gate.wait(10)
            return super().decide(state, questions, **budgets)

    s = DecisionApp({"tiny": Slow()}, "tiny", max_concurrent=1)
    t = threading.Thread(target=post, args=(s, "/v1/systemone", {"state": "x", "questions": QUESTIONS}))
    t.start()
    assert entered.wait(10)
    r = post(s, "/v1/systemone", {"state": "y", "questions": QUESTIONS})
    assert r.status == 503 and r.headers["Retry-After"] == "1"
    gate.set()
    t.join(10)


def test_http_round_trip() -> None:
    server = make_server(DecisionApp({"tiny": FakeDecider()}, "tiny"), "127.0.0.1", 0)
    thread = threading.Thread(target=server.serve_forever, daemon=True)
    thread.start()
    try:
        host, port = server.server_address[:2]
        conn = http.client.HTTPConnection(host, port, timeout=10)
        conn.request("POST", "/v1/systemone", json.dumps({"state": "x", "questions": QUESTIONS}),
                     {"Content-Type": "application/json"})
        r = conn.getresponse()
        body = json.loads(r.read())
        assert r.status == 200 and body["answers"]["mood"]["choice"] == "pos"
        for length, status in ((None, 411), ("-5", 400), ("abc", 400), (str(contract.MAX_BODY_BYTES + 1), 413)):
            conn.close()
            conn.putrequest("POST", "/v1/systemone")
            if length is not None:
                conn.putheader("Content-Length", length)
            conn.endheaders()  # no body follows: a refused body is never read
            r = conn.getresponse()
            assert r.status == status, (length, r.status)
            assert isinstance(json.loads(r.read())["detail"], str)
        conn.close()
        conn.request("GET", "/health")
        r = conn.getresponse()
        assert r.status == 200 and json.loads(r.read()) == {"status": "ok", "loaded": ["tiny"],
                                                            "default_model": "tiny", "device": "unknown"}
        conn.close()
    finally:
        server.shutdown()
        server.server_close()


def test_stalled_body_times_out(monkeypatch: pytest.MonkeyPatch) -> None:
    """A client that declares a body and stops sending it loses its connection after the handler's
    socket timeout, instead of holding the server thread; other clients are served meanwhile."""
    import socket

    from deciax_amd.serve import wsgi

    monkeypatch.setattr(wsgi._Handler, "timeout", 0.5)
    server = make_server(DecisionApp({"tiny": FakeDecider()}, "tiny"), "127.0.0.1", 0)
    thread = threading.Thread(target=server.serve_forever, daemon=True)
    thread.start()
    try:
        host, port = server.server_address[:2]
        stalled = socket.create_connection((host, port), timeout=10)
        stalled.sendall(b"POST /v1/systemone HTTP/1.1\r\nHost: x\r\nContent-Length: 100\r\n\r\n{\"questions\"")
        conn = http.client.HTTPConnection(host, port, timeout=10)
        conn.request("GET", "/health")
        assert conn.getresponse().status == 200
        conn.close()
        started = time.monotonic()
        received = b""
        while True:  # the server answers the timed-out read with an error and closes the connection
            chunk = stalled.recv(4096)
            if not chunk:
                break
            received += chunk
        assert time.monotonic() - started < 8
        assert not received or received.startswith(b"HTTP/1.") and b" 200 " not in received.split(b"\r\n", 1)[0]
        stalled.close()
    finally:
        server.shutdown()
        server.server_close()


def test_cli_choices_and_environment(monkeypatch: pytest.MonkeyPatch) -> None:
    from deciax_amd.serve.__main__ import IMPLS, parse

    assert "hip" in IMPLS and set(IMPLS) >= {"auto", "jax", "pallas"}
    args = parse(["--impl", "hip", "--model", "tiny", "--port", "0"])
    assert args.impl == "hip" and args.models == ["tiny"]
    with pytest.raises(SystemExit):
        parse(["--impl", "cuda"])
    with pytest.raises(SystemExit):
        parse(["--model", "clef"])
    monkeypatch.setenv("DECIAX_IMPL", "triton")
    with pytest.raises(SystemExit):
        parse([])
    monkeypatch.setenv("DECIAX_IMPL", "hip")
    monkeypatch.setenv("DECIAX_MODELS", "tiny,gemma2-27b")
    args = parse(["--default-model", "gemma2-27b"])
    assert args.impl == "hip" and args.models == ["tiny", "gemma2-27b"]
    with pytest.raises(SystemExit):
        parse(["--default-model", "gemma2-9b"])


def test_cli_without_a_gfx950_device_refuses_hip() -> None:
    import torch

    from deciax_amd.serve.__main__ import main

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible; the GPU test serves for real")
    with pytest.raises(ValueError, match="gfx950"):
        main(["--impl", "hip", "--model", "tiny", "--no-warmup", "--port", "0"])


def test_refusal_order_follows_the_contract() -> None:
    """Where a request breaks several rules, the contract names the one reported."""
    s = DecisionApp({"tiny": FakeDecider()}, "tiny")
    many = {f"q{i}": {"type": "choice", "criteria": {str(j): "o" for j in range(101)}} for i in range(65)}
    # more than 64 questions is reported before any per-question cap
    assert post(s, "/v1/systemone", {"state": "x", "questions": many}).payload["detail"].startswith("too many questions")
    # a score question over its level cap is reported before its null level
    over = {"s": {"type": "score", "criteria": [None] * 33}}
    assert post(s, "/v1/systemone", {"state": "x", "questions": over}).status == 413
    # limits come before refused fields, refused fields before the encoding check, that before budgets
    r = post(s, "/v1/systemone", {"state": "x" * 50001, "questions": QUESTIONS, "hooks": 1})
    assert r.status == 413
    r = post(s, "/v1/systemone", {"state": "\ud800", "questions": QUESTIONS, "lang": "en", "max_len": 0})
    assert r.status == 422 and "lang" in r.payload["detail"]
    r = post(s, "/v1/systemone", {"state": "\ud800", "questions": QUESTIONS, "max_len": 0})
    assert r.status == 400
    # a surrogate in a key is caught as well as in a value
    r = post(s, "/v1/systemone", {"state": {"\udfff": 1}, "questions": QUESTIONS})
    assert r.status == 400 and r.payload["detail"] == contract.SURROGATE_DETAIL
    # too many options across questions, each within its own cap
    spread = {f"c{i}": {"type": "choice", "criteria": [str(j) for j in range(90)]} for i in range(6)}
    r = post(s, "/v1/systemone", {"state": "x", "questions": spread})
    assert r.status == 413 and "across questions (540 > 512)" in r.payload["detail"]


def test_strict_view_and_confidence_tables_cover_every_answer_type() -> None:
    assert set(contract.STRICT_FIELDS) == {"choice", "score", "noul"}
    assert set(contract.CONFIDENCE) == {"choice", "score"}
    # score levels are ordered by their integer key, not by insertion order
    assert contract.confidence({"type": "score", "probabilities": {"2": 0.0, "0": 0.0, "1": 1.0}}) == 1.0
    assert contract.confidence({"type": "score", "probabilities": {"a": 0.5, "b": 0.5}}) is None
    # zero total mass counts as uniform
    assert contract.confidence({"type": "choice", "probabilities": {"a": 0.0, "b": 0.0}}) == 0.0
