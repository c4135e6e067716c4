"""`/v1/systemone` over the HIP decision path, as a WSGI application (PEP 3333).

Routes: `POST /v1/systemone`, `POST /v1/systemone/batch`, `GET /health`; the status codes and bodies
are the reference server's (src/deciax/serve/app.py:100-388), see `contract`. The design is this
package's own:

* `DecisionApp.respond(method, path, headers, body)` is the whole protocol, free of any HTTP framework;
  `DecisionApp.__call__` adapts it to WSGI, and `make_server` serves it on the standard library's
  WSGI server with one thread per connection.
* A decision endpoint is a fixed pipeline of stages over a `Call` record (parse, shape, model, limits,
  fields, encoding, budgets), each stage either filling the record or raising a `contract.Refusal`;
  the stage order is the contract's refusal order.
* Admission is a counter of requests in flight; past `max_concurrent` a request is refused with 503
  before any parsing. Each model's own lock serialises its device forward.
"""

from __future__ import annotations

import json
import logging
import secrets
import socketserver
import threading
import time
from collections.abc import Callable, Iterator, Mapping
from contextlib import contextmanager
from dataclasses import dataclass, field
from http import HTTPStatus
from pathlib import Path
from typing import Any
from wsgiref.simple_server import WSGIRequestHandler, WSGIServer

from deciax_amd.serve import contract
from deciax_amd.serve.contract import Refusal

log = logging.getLogger("deciax_amd.serve")

DEFAULT_TOKEN_CAP = 16384


@dataclass(frozen=True)
class Reply:
    status: int
    payload: Any
    headers: dict[str, str] = field(default_factory=dict)


def _refused(r: Refusal, headers: dict[str, str] | None = None) -> Reply:
    return Reply(r.status, {"detail": r.detail}, headers or {})


@dataclass
class Call:
    """One decision request as the pipeline fills it in."""

    raw: bytes
    batch: bool
    body: dict[str, Any] = field(default_factory=dict)
    model: str = ""
    budgets: dict[str, int] = field(default_factory=dict)


class _Admission:
    """At most `limit` requests in flight; `enter()` refuses the one past it with 503."""

    def __init__(self, limit: int) -> None:
        if limit < 1:
            raise ValueError("max_concurrent must be at least 1")
        self._limit, self._inflight, self._lock = limit, 0, threading.Lock()

    @contextmanager
    def enter(self) -> Iterator[None]:
        with self._lock:
            full = self._inflight >= self._limit
            if not full:
                self._inflight += 1
        if full:
            raise Refusal(503, "server busy, try again later")
        try:
            yield
        finally:
            with self._lock:
                self._inflight -= 1


class DecisionApp:
    """The `/v1/systemone` protocol over loaded deciders (objects with `decide` and `decide_batch`)."""

    def __init__(self, deciders: Mapping[str, Any], default_model: str, *, api_key: str | None = None,
                 max_concurrent: int = 16, jev_strict: bool = False, device: str = "unknown") -> None:
        if default_model not in deciders:
            raise ValueError(f"default model {default_model!r} is not loaded")
        self.deciders = dict(deciders)
        self.default_model = default_model
        self.device = device
        self._bearer = f"Bearer {api_key}".encode() if api_key else None
        self._admission = _Admission(max_concurrent)
        self._decorate = contract.strict_view if jev_strict else contract.with_confidence
        # route -> (method, handler, needs the bearer token and an admission slot)
        self._routes: dict[str, tuple[str, Callable[[bytes, str | None], Reply], bool]] = {
            "/health": ("GET", self._health, False),
            "/v1/systemone": ("POST", lambda raw, _auth: self._decide(Call(raw, batch=False)), True),
            "/v1/systemone/batch": ("POST", lambda raw, _auth: self._decide(Call(raw, batch=True)), True),
        }

    # ------------------------------------------------------------------ protocol core

    def respond(self, method: str, path: str, headers: Mapping[str, str], body: bytes) -> Reply:
        """The reply to one request; `headers` keys are lower case."""
        route = self._routes.get(path.split("?", 1)[0].rstrip("/") or "/")
        if route is None:
            return _refused(Refusal(404, "Not Found"))
        allowed, handler, guarded = route
        if method != allowed:
            return _refused(Refusal(405, "Method Not Allowed"))
        auth = headers.get("authorization")
        if not guarded:
            return handler(body, auth)
        if not self.authorized(auth):
            return _refused(Refusal(401, "invalid or missing bearer token"))
        try:
            with self._admission.enter():
                return handler(body, auth)
        except Refusal as r:
            return _refused(r, {"Retry-After": "1"} if r.status == 503 else None)

    def authorized(self, authorization: str | None) -> bool:
        """True when no token is configured or the header carries it (constant-time comparison)."""
        if self._bearer is None:
            return True
        return secrets.compare_digest((authorization or "").encode("utf-8", "surrogateescape"), self._bearer)

    def _health(self, _raw: bytes, auth: str | None) -> Reply:
        if not self.authorized(auth):
            return Reply(200, {"status": "ok"})
        return Reply(200, {"status": "ok", "loaded": sorted(self.deciders), "default_model": self.default_model,
                           "device": self.device})

    # ------------------------------------------------------------------ decision pipeline

    def _stage_parse(self, call: Call) -> None:
        if len(call.raw) > contract.MAX_BODY_BYTES:
            raise Refusal(413, "request body too large")
        try:
            body = json.loads(call.raw)
        except (ValueError, RecursionError):
            raise Refusal(400, "request body must be valid JSON") from None
        need = ("states", "questions") if call.batch else ("questions",)
        if not isinstance(body, dict) or any(k not in body for k in need):
            fields = "'states' and 'questions' fields" if call.batch else "a 'questions' field"
            raise Refusal(400, f"request body must be an object with {fields}")
        call.body = body

    def _stage_model(self, call: Call) -> None:
        call.model = self.model_for(call.body.get("model"))

    def _stage_limits(self, call: Call) -> None:
        b = call.body
        refusals = (contract.batch_refusals(b["states"], b["questions"]) if call.batch
                    else contract.request_refusals(b.get("state"), b["questions"]))
        contract.first(refusals)

    def _stage_fields(self, call: Call) -> None:
        unsupported = contract.UNSUPPORTED_FIELDS + (contract.UNSUPPORTED_BATCH_FIELDS if call.batch else ())
        contract.first(contract.field_refusals(call.body, unsupported))

    def _stage_encoding(self, call: Call) -> None:
        if contract.has_lone_surrogate(call.body):
            raise Refusal(400, contract.SURROGATE_DETAIL)

    def _stage_budgets(self, call: Call) -> None:
        model = getattr(self.deciders[call.model], "model", None)
        call.budgets = contract.budgets(call.body, int(getattr(model, "max_token_budget", DEFAULT_TOKEN_CAP)))

    PIPELINE = ("_stage_parse", "_stage_model", "_stage_limits", "_stage_fields", "_stage_encoding",
                "_stage_budgets")

    def _decide(self, call: Call) -> Reply:
        try:
            for stage in self.PIPELINE:
                getattr(self, stage)(call)
            decider, b = self.deciders[call.model], call.body
            started = time.perf_counter()
            try:
                if call.batch:
                    out = decider.decide_batch(b["states"], b["questions"], **call.budgets)
                else:
                    out = decider.decide(b.get("state"), b["questions"], **call.budgets)
            except ValueError as e:  # the model rejects the request (its schema, its token budget)
                raise Refusal(422, str(e)) from None
            except Refusal:
                raise
            except Exception:
                log.exception("inference failed")
                raise Refusal(500, "inference failed") from None
            ms = (time.perf_counter() - started) * 1e3
        except Refusal as r:
            return _refused(r)
        timing = {"Server-Timing": f"inference;dur={ms:.2f}", "X-Inference-Time-Ms": f"{ms:.2f}"}
        if not call.batch:
            return Reply(200, self._decorate(out), timing)
        total = {k: sum(r["usage"].get(k, 0) for r in out) for k in ("input_tokens", "output_tokens")}
        return Reply(200, {"results": [self._decorate(r) for r in out], "total_usage": total}, timing)

    def model_for(self, requested: Any) -> str:
        """The loaded model a request's `model` field selects. Absent or unknown names let the server
        choose (the default model); a loaded name selects it; a registered shape this server has not
        loaded, or anything that looks like a path, is refused with 422."""
        text = str(requested).strip() if requested else ""
        if not text:
            return self.default_model
        if text in self.deciders:
            return text
        from deciax_amd.gemma import CONFIGS

        served = sorted(self.deciders)
        if text in CONFIGS:
            raise Refusal(422, f"model {text!r} is not loaded; this server serves {served}")
        if text[:1] in ".~" or any(sep in text for sep in "/\\"):
            raise Refusal(422, f"unknown model {text!r}; this server serves {served}, "
                               "or omit model to let the server choose")
        return self.default_model

    # ------------------------------------------------------------------ WSGI adapter

    def __call__(self, environ: dict[str, Any], start_response: Callable[..., Any]) -> list[bytes]:
        method = environ.get("REQUEST_METHOD", "GET")
        body, problem = b"", None
        if method == "POST":
            body, problem = _read_body(environ)
        if problem is not None:
            reply = _refused(problem)
        else:
            headers = {"authorization": environ["HTTP_AUTHORIZATION"]} if "HTTP_AUTHORIZATION" in environ else {}
            reply = self.respond(method, environ.get("PATH_INFO") or "/", headers, body)
        data = json.dumps(reply.payload, ensure_ascii=False).encode("utf-8")
        head = [("Content-Type", "application/json"), ("Content-Length", str(len(data))), *reply.headers.items()]
        start_response(f"{reply.status} {HTTPStatus(reply.status).phrase}", head)
        return [data]


def _read_body(environ: Mapping[str, Any]) -> tuple[bytes, Refusal | None]:
    """The request body of a POST, or the refusal its Content-Length earns (411 absent, 400 not a
    non-negative integer, 413 above the body cap); a refused body is never read."""
    declared = str(environ.get("CONTENT_LENGTH") or "").strip()
    if not declared:
        return b"", Refusal(411, "Content-Length required")
    try:
        n = int(declared)
    except ValueError:
        n = -1
    if n < 0:
        return b"", Refusal(400, "invalid Content-Length")
    if n > contract.MAX_BODY_BYTES:
        return b"", Refusal(413, "request body too large")
    return environ["wsgi.input"].read(n), None


class _Handler(WSGIRequestHandler):
    # A client that declares a body and then stalls would otherwise hold its connection's thread for good
    # (the admission counter only covers requests whose body has arrived): reads and writes on the socket
    # time out after this many seconds and the connection is dropped.
    timeout = 60

    def log_message(self, format: str, *args: Any) -> None:  # noqa: A002
        log.info("%s - %s", self.address_string(), format % args)


class _ThreadingServer(socketserver.ThreadingMixIn, WSGIServer):
    daemon_threads = True


def make_server(app: DecisionApp, host: str = "127.0.0.1", port: int = 8000) -> WSGIServer:
    """A bound WSGI server for `app`, not yet serving (port 0 picks a free port); one thread per
    connection, and each response closes its connection."""
    server = _ThreadingServer((host, port), _Handler)
    server.set_app(app)
    return server


WARMUP_STATE = "warmup"
WARMUP_QUESTIONS = {"q": {"type": "noul", "instructions": "Is this a warmup request?"}}


def load_deciders(models: tuple[str, ...], *, dtype: str = "auto", impl: str = "auto",
                  seed: int = 0, warmup: bool = True) -> dict[str, Any]:
    """Load each model (a registered shape or a checkpoint directory) on the GPU, keyed by its name
    (a directory by its last path component), and run one warm-up decision through each."""
    from deciax_amd.decider import load

    out: dict[str, Any] = {}
    for name in models:
        log.info("loading %s", name)
        key = Path(name).name if Path(name).is_dir() else name
        out[key] = load(name, dtype=dtype, impl=impl, seed=seed)  # type: ignore[arg-type]
        if warmup:
            out[key].decide(WARMUP_STATE, WARMUP_QUESTIONS)
    return out


def serve(host: str = "127.0.0.1", port: int = 8000, models: tuple[str, ...] = ("gemma2-9b",), *,
          default_model: str | None = None, api_key: str | None = None, max_concurrent: int = 16,
          jev_strict: bool = False, warmup: bool = True, dtype: str = "auto", impl: str = "auto",
          seed: int = 0) -> None:
    """Load the models and serve until interrupted (the reference's `serve`, src/deciax/serve/app.py:391-423)."""
    from deciax_amd.backend import hip_device_arch

    deciders = load_deciders(models, dtype=dtype, impl=impl, seed=seed, warmup=warmup)
    app = DecisionApp(deciders, default_model or next(iter(deciders)), api_key=api_key,
                      max_concurrent=max_concurrent, jev_strict=jev_strict, device=hip_device_arch() or "unknown")
    server = make_server(app, host, port)
    log.info("serving %s on http://%s:%d", sorted(deciders), *server.server_address[:2])
    try:
        server.serve_forever()
    finally:
        server.server_close()
