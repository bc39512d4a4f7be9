"""SigLIP2 embedding service over libs2x: the reference's siglip2-server
(src/siglip2_server.cpp) with its subprocess GPU worker
(src/worker_ipc.cpp, src/worker_session.cpp).

    python -m s2x_serve --model <gguf> --tokenizer <spm.model> [--port 8890]

Endpoints (the reference's, same request and response shapes):
    GET  /health
    POST /unload, /v1/admin/unload, /v1/admin/load
    POST /v1/embeddings                 multipart `images` (+ pooling, max_num_patches)
    POST /v1/text_embeddings            form `prompts`
    POST /v1/classify                   multipart `images` + `prompts`
    POST /v1/classify_from_embeddings   JSON {image_embeddings, prompts, return_logits}

By default the GPU work runs in a child process (s2x_serve.worker) that
owns every GPU resource; /v1/admin/unload kills it, which returns all its
device memory, and the next request starts a new one.  The HTTP process
itself loads no GPU library: importing this package imports neither libs2x
nor torch (s2x_serve.engine, which does, is imported by the worker, or by
the server in in-process mode, SIGLIP2_WORKER_ISOLATION=0).
"""
