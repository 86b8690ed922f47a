// Exception-to-return-code guard shared by the extern "C" entry points.
#pragma once

#include <new>
#include <string>

#include "../../include/julia1_hip.h"
#include "common.hpp"

inline std::string& jh_error_slot() {
    thread_local std::string msg;
    return msg;
}

template <class F>
int jh_guarded(F&& f) {
    try {
        f();
        jh_error_slot().clear();
        return JH_OK;
    } catch (const jh_error& e) {
        jh_error_slot() = e.what();
        return e.code;
    } catch (const std::bad_alloc&) {
        jh_error_slot() = "host allocation failed";
        return JH_ERR_ALLOC;
    } catch (const std::exception& e) {
        jh_error_slot() = e.what();
        return JH_ERR_INTERNAL;
    } catch (...) {
        jh_error_slot() = "unknown error";
        return JH_ERR_INTERNAL;
    }
}
