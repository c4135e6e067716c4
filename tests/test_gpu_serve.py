"""`python -m deciax_amd.serve --impl hip` on the GPU: the service loads the tiny model through the
HIP path and answers over HTTP exactly what the Decider answers directly."""

from __future__ import annotations

import http.client
import json
import threading

import pytest

from tests.conftest import say

pytestmark = pytest.mark.gpu

QUESTIONS = {"sentiment": {"type": "choice", "criteria": {"pos": "positive", "neg": "negative", "neu": "neutral"}},
             "urgent": {"type": "noul"},
             "stars": {"type": "score", "criteria": ["bad", "ok", "good"]}}


def test_http_service_with_impl_hip() -> None:
    from deciax_amd.serve.__main__ import parse
    from deciax_amd.serve.contract import with_confidence
    from deciax_amd.serve.wsgi import DecisionApp, load_deciders, make_server

    say("serve --impl hip --model tiny over HTTP")
    args = parse(["--impl", "hip", "--model", "tiny", "--port", "0", "--no-warmup"])
    deciders = load_deciders(tuple(args.models), dtype=args.dtype, impl=args.impl, warmup=True)
    server = make_server(DecisionApp(deciders, "tiny", device="gfx950"), "127.0.0.1", 0)
    thread = threading.Thread(target=server.serve_forever, daemon=True)
    thread.start()
    try:
        conn = http.client.HTTPConnection(*server.server_address[:2], timeout=120)

        def call(path: str, body: dict) -> tuple[int, dict]:
            conn.request("POST", path, json.dumps(body), {"Content-Type": "application/json"})
            r = conn.getresponse()
            return r.status, json.loads(r.read())

        status, one = call("/v1/systemone", {"state": "the parcel arrived late", "questions": QUESTIONS})
        assert status == 200
        assert one == with_confidence(deciders["tiny"].decide("the parcel arrived late", QUESTIONS))
        status, batch = call("/v1/systemone/batch", {"states": ["a", {"ticket": 7}], "questions": QUESTIONS,
                                                     "max_len": 2048})
        assert status == 200 and len(batch["results"]) == 2
        assert batch["results"][0]["answers"]["sentiment"]["choice"] in ("pos", "neg", "neu")
        assert "x_jev_confidence" in batch["results"][0]["answers"]["stars"]
        status, err = call("/v1/systemone", {"state": "x", "questions": {"q": {"type": "bogus"}}})
        assert status == 422, err
        conn.close()
    finally:
        server.shutdown()
        server.server_close()
